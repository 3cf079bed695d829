"""Real-format weights into the DiT runner's reference form, against the oracle.

- Anima: two synthetic blkNN.bin files (blk_wlayout.h: fp16 crouton tiles or q8 records, gains, adaLN modulation
  weights) through hxa_dit_load_block and a synthetic small.bin (phone/extract_small.py format, with the 68-column
  x_embedder whose 4 mask-channel columns multiply zeros, animad.cpp:446, and an LLM-adapter tensor the loader skips)
  through hxa_dit_load_anima_glue; one velocity against oracle_anima_ref_velocity built from the same files.
- MOSS: a synthetic glue.bin (MGL1, moss/export_glue.py) with the reference's storage types (fp32 time MLP, video
  embedding, head linear, vectors; fp16 modulation matrices) and non-default RoPE bands through
  hxa_dit_load_moss_glue; the DiT's exported glue sections must equal the file's tensors bit for bit, then four
  rapid-moss steps with the file's step codes against oracle_moss_rapid_step on the file's tensors.

The modulation weights are large enough that the gates are O(0.1 - 1): how much the blocks change the output is
printed and bounded below, so a block loaded into the wrong place fails. Tolerance about 3x the error measured on
MI355X."""
import ctypes as C
import struct

import numpy as np
import pytest

from oracle import hxo
from tests._helpers import (bn_unpatchify, f16, moss_ref_sections, oracle_anima_ref_velocity, oracle_moss_rapid_step,
                            rel, split_flat, unpack_weights)
from tests.test_gpu_block import W_MODW, W_TOTAL, _blk_file, _export

pytestmark = pytest.mark.gpu


def _hip():
    from hexanima_amd import hip
    hip.init()
    return hip


def small_bin(tensors):
    """phone/extract_small.py's format: u32 count; per tensor u32 name length, name, u32 ndim, i64 dims, fp16 data."""
    out = [struct.pack("<I", len(tensors))]
    for name, a in tensors:
        a = np.ascontiguousarray(a, np.float16)
        out.append(struct.pack("<I", len(name)) + name.encode() + struct.pack("<I", a.ndim) +
                   struct.pack(f"<{a.ndim}q", *a.shape) + a.tobytes())
    return np.frombuffer(b"".join(out), np.uint8).copy()


def mgl1_bin(tensors):
    """moss/export_glue.py's format: "MGL1", i32 n; n x {char name[40]; i32 dtype (0 f32, 1 f16); i32 nd; i32 dims[3];
    i64 offset; i64 bytes}; data 128-byte aligned."""
    hdr = 8 + len(tensors) * 76
    off = (hdr + 127) // 128 * 128
    ent, data = b"", []
    for name, dt, a in tensors:
        d = list(a.shape) + [1] * (3 - a.ndim)
        ent += struct.pack("<40sii3iqq", name.encode(), dt, a.ndim, *d, off, a.nbytes)
        data.append((off, a.tobytes()))
        off = (off + a.nbytes + 127) // 128 * 128
    buf = bytearray(off)
    buf[:hdr] = b"MGL1" + struct.pack("<i", len(tensors)) + ent
    for o, b in data:
        buf[o:o + len(b)] = b
    return np.frombuffer(bytes(buf), np.uint8).copy()


# 256 image tokens, and the benchmark's 1536 (a 96 x 64 latent; int8 blocks then take the fused split-K 4 form)
@pytest.mark.parametrize("q8,LAT", [(False, (16, 32, 32)), (True, (16, 32, 32)), (False, (16, 96, 64)),
                                    (True, (16, 96, 64))])
def test_dit_anima_from_blk_files_and_small_bin(q8, LAT):
    hip = _hip()
    lib = hip.lib()
    hxo.set_threads(0)
    D, H, F, CT, DC, NB, C4 = 2048, 16, 8192, 512, 1024, 2, 64
    print(f"[case] DiT from 2 blkNN.bin ({'q8' if q8 else 'fp16'}) + small.bin, {LAT[1] * LAT[2] // 4} tokens",
          flush=True)
    fmt = hip.W_Q8 if q8 else hip.W_F16
    bd = hip.BlockDims(0, D, H, F, CT, DC, 0, 1, 0, fmt, fmt, 0)
    cfg = hip.DitCfg(bd, NB, LAT[0], LAT[1], LAT[2], D, 0, 1)
    p = C.c_void_p()
    hip.check(lib.hxa_dit_create(C.byref(cfg), 4242, C.byref(p)), "dit_create")
    try:
        rng = np.random.default_rng(91 + q8)
        blocks, modws = [], []
        for k in range(NB):
            buf, ow = _blk_file(rng, q8, modw=True)
            hip.check(lib.hxa_dit_load_block(p, k, buf.ctypes.data, buf.nbytes), "load_block")
            blocks.append(ow)
            moff = W_MODW if not q8 else 125829120 // 2048 * 1152 + 4096
            mw = buf[moff:moff + (W_TOTAL - W_MODW)].view(np.uint16).reshape(3, 256 * D + 3 * D * 256)
            modws.append((np.ascontiguousarray(mw[:, :256 * D]).reshape(768, D),
                          np.ascontiguousarray(mw[:, 256 * D:]).reshape(3, 3 * D, 256)))
        w = lambda *sh: f16(rng.standard_normal(sh) * 0.02)
        xemb = w(D, C4 + 4)
        glue = [("llm_adapter.in_proj.weight", w(32, 16)),
                ("t_embedder.1.linear_1.weight", w(D, D)), ("t_embedder.1.linear_2.weight", w(3 * D, D)),
                ("t_embedding_norm.weight", f16(1 + 0.1 * rng.standard_normal(D))),
                ("x_embedder.proj.1.weight", xemb),
                ("final_layer.adaln_modulation.1.weight", w(256, D)),
                ("final_layer.adaln_modulation.2.weight", w(2 * D, 256)), ("final_layer.linear.weight", w(C4, D))]
        sb = small_bin(glue)
        hip.check(lib.hxa_dit_load_anima_glue(p, sb.ctypes.data, sb.nbytes), "load_anima_glue")
        assert lib.hxa_dit_load_anima_glue(p, sb.ctypes.data, sb.nbytes - 7) == -5  # truncated: HXA_E_WEIGHTS
        g = dict(glue)
        u = lambda a: np.ascontiguousarray(a).view(np.uint16)
        oglue = (u(xemb[:, :C4]), u(g["t_embedder.1.linear_1.weight"]), u(g["t_embedder.1.linear_2.weight"]),
                 u(g["final_layer.adaln_modulation.1.weight"]), u(g["final_layer.adaln_modulation.2.weight"]),
                 u(g["final_layer.linear.weight"]), u(g["t_embedding_norm.weight"]))
        lat = rng.standard_normal((1,) + LAT).astype(np.float32)
        ctx = rng.standard_normal((1, CT, DC)).astype(np.float32)
        hip.check(lib.hxa_dit_set_inputs(p, lat.ctypes.data, ctx.ctypes.data), "set_inputs")
        v = np.zeros_like(lat)
        hip.check(lib.hxa_dit_velocity(p, 0.75, v.ctypes.data), "velocity")
        kw = dict(D=D, H=H, F=F, C4=C4, gelu=0)
        ref = oracle_anima_ref_velocity(lat, f16(ctx), 0.75, blocks, modws, oglue, **kw)
        ref0 = oracle_anima_ref_velocity(lat, f16(ctx), 0.75, [], [], oglue, **kw)
        share = rel(ref, ref0)
        r, mx = rel(v, ref), float(np.max(np.abs(v - ref)))
        print(f"velocity rel err {r:.3e} max abs {mx:.3e}; the blocks change it by {share:.3f} (relative)", flush=True)
        assert share > 0.2  # measured 1.20 / 1.11 (256 tokens), 1.19 / 1.12 (1536)
        # measured 6.0e-4 / 6.5e-4, 2.8e-3 / 2.5e-3 (fp16 / q8, 256 tokens); 5.9e-4 / 6.4e-4, 3.1e-3 / 2.9e-3 (1536)
        assert r < 2e-3 and mx < 9e-3
    finally:
        lib.hxa_dit_destroy(p)


def test_dit_moss_from_mgl1_glue():
    hip = _hip()
    lib = hip.lib()
    D, H, F, ntxt, tin, nb, B = 256, 2, 512, 20, 128, 2, 1
    C4, LAT = 128, (32, 16, 16)
    print("[case] MOSS DiT reference form with glue.bin (MGL1), 2 blocks, 4 rapid-moss steps", flush=True)
    bd = hip.BlockDims(1, D, H, F, ntxt, 0, 0, B, 0, hip.W_Q8, hip.W_Q4, 1)
    cfg = hip.DitCfg(bd, nb, LAT[0], LAT[1], LAT[2], 256, tin, 1)
    p = C.c_void_p()
    hip.check(lib.hxa_dit_create(C.byref(cfg), 4343, C.byref(p)), "dit_create")
    try:
        rng = np.random.default_rng(93)
        f32 = lambda *sh, s=0.02, m=0.0: (m + s * rng.standard_normal(sh)).astype(np.float32)
        bands = (1.3 / 10000.0 ** (np.arange(16) / 16.0)).astype(np.float32)
        # a small video embedding and a large time MLP output: the gates are O(0.5) and the blocks' updates are of
        # the size of the embedded tokens
        t = [("video_embedder.weight", 0, f32(D, C4, s=0.005)), ("video_embedder.bias", 0, f32(D, s=0.005)),
             ("time_embedding.0.weight", 0, f32(D, 256)), ("time_embedding.0.bias", 0, f32(D)),
             ("time_embedding.2.weight", 0, f32(D, D, s=0.2)), ("time_embedding.2.bias", 0, f32(D)),
             ("shared_block_modulation.weight", 1, f16(rng.standard_normal((6 * D, D)) * 0.16)),
             ("shared_block_modulation.bias", 0, f32(6 * D)),
             ("video_head_modulation.weight", 1, f16(rng.standard_normal((2 * D, D)) * 0.02)),
             ("video_head_modulation.bias", 0, f32(2 * D)),
             ("final_linear_video.weight", 0, f32(C4, D)), ("final_norm_video.weight", 0, f32(D, s=0.1, m=1.0)),
             ("latent_mix.Q", 0, f32(C4, C4)), ("step_codes", 0, np.array([0.999, 0.75, 0.5, 0.25], np.float32)),
             ("rope.bands", 0, bands), ("bn.mean", 0, f32(C4, s=0.1)), ("bn.var", 0, f32(C4, s=0.1, m=1.0))]
        gb = mgl1_bin(t)
        hip.check(lib.hxa_dit_load_moss_glue(p, gb.ctypes.data, gb.nbytes), "load_moss_glue")
        bad = gb.copy()
        bad[:4] = np.frombuffer(b"MGL0", np.uint8)
        assert lib.hxa_dit_load_moss_glue(p, bad.ctypes.data, bad.nbytes) == -5  # HXA_E_WEIGHTS
        g = {n: a for n, _, a in t}
        # the loaded sections, bit for bit
        glue16 = _export(hip, p, 2 * nb).view(np.uint16)
        vec32 = _export(hip, p, 2 * nb + 1).view(np.float32)
        Wh, Wt = split_flat(glue16, [(2 * D, D), (D, tin)])
        assert np.array_equal(Wh, g["video_head_modulation.weight"].view(np.uint16))
        v = split_flat(vec32, [(D,), (D,), (D,), (6 * D,), (2 * D,), (D,), (C4, C4), (C4,), (C4,), (D, C4), (D, 256),
                               (D, D), (C4, D)])
        names = ["video_embedder.bias", "time_embedding.0.bias", "time_embedding.2.bias", "shared_block_modulation.bias",
                 "video_head_modulation.bias", "final_norm_video.weight", "latent_mix.Q", "bn.mean", "bn.var",
                 "video_embedder.weight", "time_embedding.0.weight", "time_embedding.2.weight",
                 "final_linear_video.weight"]
        for a, n in zip(v, names):
            assert np.array_equal(a, g[n]), n
        modw = _export(hip, p, nb).view(np.uint16).reshape(6 * D, D)
        assert np.array_equal(modw, g["shared_block_modulation.weight"].view(np.uint16))
        layout = hip.pack_layout(1, D, F, 0, hip.W_Q8, hip.W_Q4)
        blocks = [unpack_weights(_export(hip, p, k), 1, D, F, 0, hip.W_Q8, hip.W_Q4, layout) for k in range(nb)]
        glue, vec = moss_ref_sections(glue16, vec32, D, C4, tin)
        z = rng.standard_normal((B,) + LAT).astype(np.float32)
        txt = rng.standard_normal((B, ntxt, tin)).astype(np.float32)
        hip.check(lib.hxa_dit_set_inputs(p, z.ctypes.data, txt.ctypes.data), "set_inputs")
        zr = np.stack([hxo.patchify(z[b]) for b in range(B)])
        x0, x00 = np.zeros_like(zr), np.zeros_like(zr)
        txt16 = f16(txt)
        kw = dict(D=D, H=H, F=F, C4=C4, ntxt=ntxt, Ttot=96, gh=8, gw=8, bands=bands)
        for code in g["step_codes"]:
            hip.check(lib.hxa_dit_moss_step(p, float(code), 1), "moss_step")
            x0 = oracle_moss_rapid_step(zr, x0, txt16, float(code), blocks, modw, glue, vec, **kw)
            x00 = oracle_moss_rapid_step(zr, x00, txt16, float(code), [], modw, glue, vec, **kw)
        got = np.zeros_like(z)
        hip.check(lib.hxa_dit_get_latent(p, got.ctypes.data), "get_latent")
        ref = np.stack([bn_unpatchify(x0[b], vec[7], vec[8], *LAT) for b in range(B)])
        share = rel(x0, x00)
        r, mx = rel(got, ref), float(np.max(np.abs(got - ref)))
        print(f"rapid-moss from glue.bin: rel err {r:.2e} max abs {mx:.2e}; the blocks change x0 by {share:.3f}",
              flush=True)
        assert share > 0.2  # measured 0.365
        assert r < 6e-4 and mx < 2.5e-3  # measured 2.0e-4, 8.2e-4
    finally:
        lib.hxa_dit_destroy(p)


def test_dit_moss_lora_blocks_from_files():
    """The MOSS DiT of LoRA blocks (kind 2): two synthetic export_moss.py block files through hxa_dit_load_moss_block
    (the conversion mega_block's MOSS path uses) and an MGL1 glue.bin at the real width (D 3072), four rapid-moss
    steps against oracle_moss_rapid_step with the files' blocks (the LoRA term included)."""
    from tests.test_gpu_block import _moss_blk_file
    hip = _hip()
    lib = hip.lib()
    hxo.set_threads(0)
    D, H, F, ntxt, tin, nb, B = 3072, 24, 8192, 20, 64, 2, 1
    C4, LAT = 128, (32, 16, 16)
    print("[case] MOSS DiT of LoRA blocks from block files + glue.bin, D 3072, 2 blocks, 4 rapid-moss steps",
          flush=True)
    bd = hip.BlockDims(2, D, H, F, ntxt, 0, 0, B, 0, hip.W_Q8, hip.W_Q8, 1)
    cfg = hip.DitCfg(bd, nb, LAT[0], LAT[1], LAT[2], 256, tin, 1)
    p = C.c_void_p()
    hip.check(lib.hxa_dit_create(C.byref(cfg), 4444, C.byref(p)), "dit_create")
    try:
        rng = np.random.default_rng(97)
        blocks = []
        for k in range(nb):
            wf, w = _moss_blk_file(rng)
            hip.check(lib.hxa_dit_load_moss_block(p, k, wf.ctypes.data, wf.nbytes), "load_moss_block")
            blocks.append(w)
        assert lib.hxa_dit_load_moss_block(p, 0, wf.ctypes.data, wf.nbytes - 1) == -5  # HXA_E_WEIGHTS (size)
        f32 = lambda *sh, s=0.02, m=0.0: (m + s * rng.standard_normal(sh)).astype(np.float32)
        bands = (1.0 / 10000.0 ** (np.arange(16) / 16.0)).astype(np.float32)
        t = [("video_embedder.weight", 0, f32(D, C4, s=0.005)), ("video_embedder.bias", 0, f32(D, s=0.005)),
             ("time_embedding.0.weight", 0, f32(D, 256)), ("time_embedding.0.bias", 0, f32(D)),
             ("time_embedding.2.weight", 0, f32(D, D)), ("time_embedding.2.bias", 0, f32(D)),
             ("shared_block_modulation.weight", 1, f16(rng.standard_normal((6 * D, D)) * 0.02)),
             ("shared_block_modulation.bias", 0, f32(6 * D)),
             ("video_head_modulation.weight", 1, f16(rng.standard_normal((2 * D, D)) * 0.02)),
             ("video_head_modulation.bias", 0, f32(2 * D)),
             ("final_linear_video.weight", 0, f32(C4, D)), ("final_norm_video.weight", 0, f32(D, s=0.1, m=1.0)),
             ("latent_mix.Q", 0, f32(C4, C4)), ("step_codes", 0, np.array([0.999, 0.75, 0.5, 0.25], np.float32)),
             ("rope.bands", 0, bands), ("bn.mean", 0, f32(C4, s=0.1)), ("bn.var", 0, f32(C4, s=0.1, m=1.0))]
        gb = mgl1_bin(t)
        hip.check(lib.hxa_dit_load_moss_glue(p, gb.ctypes.data, gb.nbytes), "load_moss_glue")
        g = {n: a for n, _, a in t}
        glue, vec = moss_ref_sections(_export(hip, p, 2 * nb).view(np.uint16),
                                      _export(hip, p, 2 * nb + 1).view(np.float32), D, C4, tin)
        modw = _export(hip, p, nb).view(np.uint16).reshape(6 * D, D)
        z = rng.standard_normal((B,) + LAT).astype(np.float32)
        txt = rng.standard_normal((B, ntxt, tin)).astype(np.float32)
        hip.check(lib.hxa_dit_set_inputs(p, z.ctypes.data, txt.ctypes.data), "set_inputs")
        zr = np.stack([hxo.patchify(z[b]) for b in range(B)])
        x0, x00 = np.zeros_like(zr), np.zeros_like(zr)
        txt16 = f16(txt)
        kw = dict(D=D, H=H, F=F, C4=C4, ntxt=ntxt, Ttot=96, gh=8, gw=8, bands=bands)
        for code in g["step_codes"]:
            hip.check(lib.hxa_dit_moss_step(p, float(code), 1), "moss_step")
            x0 = oracle_moss_rapid_step(zr, x0, txt16, float(code), blocks, modw, glue, vec, **kw)
            x00 = oracle_moss_rapid_step(zr, x00, txt16, float(code), [], modw, glue, vec, **kw)
        got = np.zeros_like(z)
        hip.check(lib.hxa_dit_get_latent(p, got.ctypes.data), "get_latent")
        ref = np.stack([bn_unpatchify(x0[b], vec[7], vec[8], *LAT) for b in range(B)])
        share = rel(x0, x00)
        r, mx = rel(got, ref), float(np.max(np.abs(got - ref)))
        print(f"MOSS LoRA DiT from files: rel err {r:.2e} max abs {mx:.2e}; the blocks change x0 by {share:.3f}",
              flush=True)
        assert share > 0.2
        assert r < 3e-3 and mx < 3e-2
    finally:
        lib.hxa_dit_destroy(p)
