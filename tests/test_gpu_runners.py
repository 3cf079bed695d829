"""GPU parity of the processes above the block ABI: the GPU modulation (megarun.cpp:156-171), hxa_run speaking
megarun's stdin protocol (megarun.cpp:132-195) and hxa_blk, the blk_main-style harness (blk_main.c:16-59). The
programs run as child processes, the way animad drives megarun (phone/animad.cpp:461-469), on synthetic blkNN.bin
files; their outputs are compared with the oracle: the modulation composed from the oracle's fp32 linear, the
blocks from hxo.anima_block with the reference's erf GELU and 512 context tokens. Tolerances as in test_gpu_block
(about 3x the error measured on MI355X)."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

from oracle import hxo
from tests._helpers import f16, oracle_anima_modulation, rel
from tests.test_gpu_block import W_MODW, W_TOTAL, _blk_file, metrics_line

pytestmark = pytest.mark.gpu
D, F, NCTX = 2048, 8192, 512


def _hip():
    from hexanima_amd import hip
    hip.init()
    return hip


def _prog(hip, name):
    # HXA_PROG_DIR: run other builds of the host programs, e.g. the AddressSanitizer + UBSan ones of
    # `python -m hexanima_amd.build --sanitize` (hexanima_amd/_san)
    p = os.path.join(os.environ.get("HXA_PROG_DIR") or os.path.dirname(hip.LIB_PATH), name)
    assert os.access(p, os.X_OK), f"{p} is not built"
    return p


def _modw(buf, q8):
    off = W_MODW if not q8 else 125829120 // 2048 * 1152 + 4096
    return buf[off:off + (W_TOTAL - W_MODW)].view(np.uint16)


@pytest.mark.parametrize("q8", [False, True])
def test_anima_modulation_matches_oracle(q8):
    """hxa_anima_modulation on two registered blkNN.bin files (fp16: W_MODW, q8: WQ_MODW, told apart by size) against
    lora + B (A silu(emb)) per site in fp32 from the same fp16 weights."""
    hip = _hip()
    print(f"[case] GPU modulation q8={q8}", flush=True)
    lib = hip.lib()
    rng = np.random.default_rng(61 + q8)
    files = [_blk_file(rng, q8, modw=True)[0] for _ in range(2)]
    emb = rng.standard_normal(D).astype(np.float32)
    lora = (rng.standard_normal(6144) * 0.1).astype(np.float32)
    h = C.c_uint64()
    hip.check(lib.mega_open(b"", C.byref(h)), "mega_open")
    try:
        for i, b in enumerate(files):
            hip.check(lib.hxa_register(h, 10 + i, b.ctypes.data, b.nbytes, hip.KIND_WEIGHTS_ANIMA), "register")
        fds = np.array([10, 11], np.int32)
        mod = np.zeros((2, 9, D), np.float32)
        hip.check(lib.hxa_anima_modulation(h, fds.ctypes.data, 2, emb.ctypes.data, lora.ctypes.data, mod.ctypes.data),
                  "modulation")
        for k in range(2):
            ref = oracle_anima_modulation(_modw(files[k], q8), emb, lora)
            e, mx = rel(mod[k], ref), float(np.max(np.abs(mod[k] - ref)))
            print(f"block {k}: modulation rel err {e:.2e} max abs {mx:.2e}", flush=True)
            assert e < 5e-7 and mx < 4e-7  # measured 1.5e-7, 1.2e-7: fp32 sums in another order
        bad = np.array([99], np.int32)
        assert lib.hxa_anima_modulation(h, bad.ctypes.data, 1, emb.ctypes.data, lora.ctypes.data, mod.ctypes.data) == -5
    finally:
        lib.mega_close(h)


@pytest.mark.parametrize("q8", [False, True])
def test_hxa_run_megarun_protocol(tmp_path, q8):
    """Two blocks through hxa_run: `run X_IN EMB LORA CTX X_OUT GH GW [SKIPMASK]` -> `done <ms>` with X [D][T]
    fp32 files, once with both blocks and once skipping block 0 (skipmask bit 0); fp16 files, and q8 files (told
    apart by size, megarun.cpp:97)."""
    hip = _hip()
    print(f"[case] hxa_run megarun protocol, 2 {'q8' if q8 else 'fp16'} blocks, T=1536", flush=True)
    rng = np.random.default_rng(71 + q8)
    blocks = []
    for i in range(2):
        buf, ow = _blk_file(rng, q8, modw=True)
        buf.tofile(tmp_path / f"blk{i:02d}.bin")
        blocks.append((buf, ow))
    gh, gw = 48, 32
    T = gh * gw
    x = rng.standard_normal((T, D)).astype(np.float32)
    emb = rng.standard_normal(D).astype(np.float32)
    lora = (rng.standard_normal(6144) * 0.1).astype(np.float32)
    ctx = rng.standard_normal((NCTX, 1024)).astype(np.float32)
    np.ascontiguousarray(x.T).tofile(tmp_path / "x_in.raw")  # megarun's [D][T] files
    emb.tofile(tmp_path / "emb.raw")
    lora.tofile(tmp_path / "lora.raw")
    np.ascontiguousarray(ctx.T).tofile(tmp_path / "ctx.raw")
    p = str(tmp_path)
    cmds = (f"run {p}/x_in.raw {p}/emb.raw {p}/lora.raw {p}/ctx.raw {p}/x_out.raw {gh} {gw}\n"
            f"run {p}/x_in.raw {p}/emb.raw {p}/lora.raw {p}/ctx.raw {p}/x_skip.raw {gh} {gw} 1\n"
            f"run {p}/x_in.raw {p}/emb.raw {p}/lora.raw {p}/missing.raw {p}/x_bad.raw {gh} {gw}\nquit\n")
    r = subprocess.run([_prog(hip, "hxa_run"), p, "0", "2"], input=cmds, capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0 and r.stdout.startswith("ready")
    out = r.stdout.splitlines()
    assert out[1].startswith("done ") and out[2].startswith("done ") and out[3] == "error", out
    cos, sin = hxo.rope_anima(gh, gw)
    ctx16 = f16(ctx)
    ref, ref1 = x, x
    for k, (buf, ow) in enumerate(blocks):
        m9 = oracle_anima_modulation(_modw(buf, q8), emb, lora)
        ref, _, _ = hxo.anima_block(ref, ctx16, m9, cos, sin, ow, H=16, F=F, gelu=0)
        if k == 1:
            ref1, _, _ = hxo.anima_block(x, ctx16, m9, cos, sin, ow, H=16, F=F, gelu=0)
    for name, want in (("x_out.raw", ref), ("x_skip.raw", ref1)):
        got = np.fromfile(tmp_path / name, np.float32).reshape(D, T).T
        r_, c, mx = metrics_line(got, want, x)
        print(f"{name}: rel err on delta {r_:.2e} cos {c:.8f} max abs {mx:.2e}", flush=True)
        assert r_ < 1.4e-3 and c > 1 - 1.4e-3 ** 2 and mx < 1e-2  # measured fp16 4.5e-4 / 3.8e-4, 2.7e-3 / 3.2e-3; q8 3.9e-4 / 3.4e-4, 2.0e-3 / 1.6e-3


def test_hxa_blk_harness(tmp_path):
    """One fp16 block through hxa_blk from export_block.py-style files (x32.bin, ctx16.bin, mod.bin, cos/sin.bin,
    w_*.bin, gain.bin): two reps print their stage times and out32.bin matches the oracle; with STOP = 4 the block
    stops before its first residual, so x comes back unchanged."""
    hip = _hip()
    print("[case] hxa_blk harness, T=1536", flush=True)
    rng = np.random.default_rng(81)
    T = 1536
    buf, ow = _blk_file(rng, False)
    offs = {"w_sq": 0, "w_sk": 8388608, "w_sv": 16777216, "w_so": 25165824, "w_cq": 33554432, "w_ck": 41943040,
            "w_cv": 46137344, "w_co": 50331648, "w_m1": 58720256, "w_m2": 92274688, "gain": 125829120}
    sizes = {"w_ck": 4194304, "w_cv": 4194304, "w_m1": 33554432, "w_m2": 33554432, "gain": 2048}
    for name, o in offs.items():
        buf[o:o + sizes.get(name, 8388608)].tofile(tmp_path / f"{name}.bin")
    x = rng.standard_normal((T, D)).astype(np.float32)
    ctx = f16(rng.standard_normal((NCTX, 1024)))
    mod = (rng.standard_normal((9, D)) * 0.2).astype(np.float32)
    cos, sin = hxo.rope_anima(48, 32)
    hxo.x32_tile(x).tofile(tmp_path / "x32.bin")
    hxo.h16_tile(ctx).tofile(tmp_path / "ctx16.bin")
    mod.tofile(tmp_path / "mod.bin")
    for nm, tab in (("cos", cos), ("sin", sin)):
        np.ascontiguousarray(tab.reshape(T // 32, 32, 2, 32).transpose(0, 2, 1, 3)).astype(np.float32).tofile(tmp_path / f"{nm}.bin")
    exe = _prog(hip, "hxa_blk")
    r = subprocess.run([exe, str(tmp_path), "2", "0", "3"], capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr, flush=True)
    reps = [l for l in r.stdout.splitlines() if l.startswith("rep ")]
    assert r.returncode == 0 and len(reps) == 2 and all(" rc=0 " in l for l in reps)
    stages = [int(v) for v in reps[1].split("|")[1].split()[1:]]
    assert len(stages) == 24 and all(v >= 0 for v in stages[:13]) and all(v == 0 for v in stages[13:23])
    got = hxo.x32_untile(np.fromfile(tmp_path / "out32.bin", np.float32), T, D)
    ref, _, _ = hxo.anima_block(x, ctx, mod, cos, sin, ow, H=16, F=F, gelu=0)
    r_, c, mx = metrics_line(got, ref, x)
    print(f"hxa_blk rel err on delta {r_:.2e} cos {c:.8f} max abs {mx:.2e}", flush=True)
    assert r_ < 1.2e-3 and c > 1 - 1.2e-3 ** 2 and mx < 7e-3  # measured 3.7e-4, 2.2e-3
    r = subprocess.run([exe, str(tmp_path), "1", "4", "3"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout
    stages = [int(v) for v in [l for l in r.stdout.splitlines() if l.startswith("rep ")][0].split("|")[1].split()[1:]]
    assert all(v == 0 for v in stages[4:17])
    assert np.array_equal(hxo.x32_untile(np.fromfile(tmp_path / "out32.bin", np.float32), T, D), x)
