"""Parity of the MOSS-class DiT at its own full shape against the oracle: latent 32 x 128 x 192 -> 6144 image tokens
(a 64 x 96 patch grid) plus 512 text tokens of width 4096 projected to 3072 into the joint token layout (6656 tokens),
hidden 3072, 24 heads, SiTU MLP 12288, int8 attention and int4 MLP weights (group 32), two blocks.

Two forms of the glue around the blocks:
- form 0 (the benchmark configuration's): one velocity v(x, 0.75), against oracle_moss_velocity;
- form 1 (the reference's rapid-moss sampler, mossrun.cpp:255-343): two steps (codes 0.999 and 0.75; the second one
  runs the latent mix on the first step's clean estimate), the BN-denormalised x0 against oracle_moss_rapid_step.

The synthetic weights are N(0, 0.02); the shared block modulation weights are scaled by 4 after creation (exported,
scaled, imported back), so that the adaLN gates are O(0.1 - 1) and the two blocks' residual updates dominate the
output: the block wiring inside the DiT (joint layout, text rows, masked padding, chained residuals) is what this
pins, where the small-width DiT tests with small gates pin mostly the glue. The mean |gate| is printed (0.40 on
both sites), and so is how much the blocks change the result: the oracle without its blocks differs from the oracle
with them by 137% (velocity) and 103% (x0) of the latter.

Tolerance about 3x the error measured on MI355X. The oracle needs about a minute on 16 host threads."""
import ctypes as C_
import time

import numpy as np
import pytest

from oracle import hxo
from tests._helpers import (bn_unpatchify, f16, moss_ref_sections, oracle_moss_rapid_step, oracle_moss_velocity, rel, silu,
                            unpack_weights)

pytestmark = pytest.mark.gpu

D, H, F, NTXT, TIN, NB = 3072, 24, 12288, 512, 4096, 2
LAT = (32, 128, 192)
C4, GH, GW = 4 * LAT[0], LAT[1] // 2, LAT[2] // 2
TIMG = GH * GW
TTOT = (TIMG + NTXT + 31) // 32 * 32
MOD_SCALE = 4.0


def _split(buf, shapes):
    out, o = [], 0
    for sh in shapes:
        n = int(np.prod(sh))
        out.append(buf[o:o + n].reshape(sh))
        o += n
    assert o == buf.size
    return out


def _make(hip, form, seed):
    lib = hip.lib()
    bd = hip.BlockDims(1, D, H, F, NTXT, 0, 0, 1, 0, hip.W_Q8, hip.W_Q4, 1)
    cfg = hip.DitCfg(bd, NB, LAT[0], LAT[1], LAT[2], 256, TIN, form)
    p = C_.c_void_p()
    hip.check(lib.hxa_dit_create(C_.byref(cfg), seed, C_.byref(p)), "dit_create")
    return p


def _export(lib, p, which):
    n = lib.hxa_dit_export(p, which, None, 0)
    buf = np.zeros(n, np.uint8)
    assert lib.hxa_dit_export(p, which, buf.ctypes.data, n) == n
    return buf


def _scaled_modw(hip, lib, p):
    """The shared modulation weights times MOD_SCALE (rounded to fp16), imported back; returns them as uint16."""
    m = _export(lib, p, NB).view(np.float16)
    m2 = f16(m.astype(np.float32) * MOD_SCALE)
    hip.check(lib.hxa_dit_import(p, NB, m2.ctypes.data, m2.nbytes), "dit_import")
    return m2.view(np.uint16).reshape(6 * D, D)


def _blocks(hip, lib, p):
    layout = hip.pack_layout(1, D, F, 0, hip.W_Q8, hip.W_Q4)
    return [unpack_weights(_export(lib, p, k), 1, D, F, 0, hip.W_Q8, hip.W_Q4, layout) for k in range(NB)]


def test_dit_moss_6656tok_velocity_vs_oracle():
    from hexanima_amd import hip

    hip.init(0)
    lib = hip.lib()
    hxo.set_threads(0)
    print(f"[case] MOSS-class DiT form 0, {NB} blocks, {TIMG}+{NTXT} tokens, q8/q4, velocity vs oracle", flush=True)
    p = _make(hip, 0, 6161)
    try:
        modw = _scaled_modw(hip, lib, p)
        rng = np.random.default_rng(61)
        lat = rng.standard_normal((1,) + LAT).astype(np.float32)
        txt = rng.standard_normal((1, NTXT, TIN)).astype(np.float32)
        hip.check(lib.hxa_dit_set_inputs(p, lat.ctypes.data, txt.ctypes.data), "set_inputs")
        v = np.zeros_like(lat)
        hip.check(lib.hxa_dit_velocity(p, 0.75, v.ctypes.data), "velocity")
        blocks = _blocks(hip, lib, p)
        glue = _split(_export(lib, p, 2 * NB).view(np.uint16), [(D, C4), (D, 256), (2 * D, D), (C4, D), (D, TIN)])
        sc = silu(hxo.linear_f32(hxo.sinusoid(0.75, 256)[None, :], glue[1]))
        mod6 = hxo.linear_f32(sc, modw)[0].reshape(6, D)
        print(f"mean |gate| attention {np.abs(mod6[2]).mean():.3f}, ffn {np.abs(mod6[5]).mean():.3f}; "
              f"mean |scale| {np.abs(mod6[[1, 4]]).mean():.3f}", flush=True)
        t0 = time.time()
        ref = oracle_moss_velocity(lat, f16(txt), 0.75, blocks, modw, glue, D=D, H=H, F=F, C4=C4, temb=256, ntxt=NTXT,
                                   Ttot=TTOT)
        print(f"oracle velocity in {time.time() - t0:.1f} s", flush=True)
        # how much the blocks move the output: the oracle velocity of the same DiT without its blocks
        ref0 = oracle_moss_velocity(lat, f16(txt), 0.75, [], modw, glue, D=D, H=H, F=F, C4=C4, temb=256, ntxt=NTXT,
                                    Ttot=TTOT)
        share = rel(ref, ref0)
        r, mx = rel(v, ref), float(np.max(np.abs(v - ref)))
        print(f"MOSS-class DiT velocity: rel err {r:.3e}, max abs {mx:.3e}; the blocks change the velocity by "
              f"{share:.3f} (relative)", flush=True)
        assert np.isfinite(v).all()
        assert share > 0.2  # the blocks' updates are a large part of the output (measured 1.37)
        assert r < 2.7e-3 and mx < 1.7e-2  # measured 9.0e-4, 5.5e-3
    finally:
        lib.hxa_dit_destroy(p)


def test_dit_moss_6656tok_rapid_steps_vs_oracle():
    from hexanima_amd import hip

    hip.init(0)
    lib = hip.lib()
    hxo.set_threads(0)
    print(f"[case] MOSS-class DiT form 1 (rapid-moss), {NB} blocks, {TIMG}+{NTXT} tokens, q8/q4, 2 steps vs oracle",
          flush=True)
    p = _make(hip, 1, 6262)
    try:
        modw = _scaled_modw(hip, lib, p)
        rng = np.random.default_rng(62)
        z = rng.standard_normal((1,) + LAT).astype(np.float32)
        txt = rng.standard_normal((1, NTXT, TIN)).astype(np.float32)
        hip.check(lib.hxa_dit_set_inputs(p, z.ctypes.data, txt.ctypes.data), "set_inputs")
        codes = [0.999, 0.75]
        for code in codes:
            hip.check(lib.hxa_dit_moss_step(p, code, 1), "moss_step")
        got = np.zeros_like(z)
        hip.check(lib.hxa_dit_get_latent(p, got.ctypes.data), "get_latent")
        blocks = _blocks(hip, lib, p)
        glue, vec = moss_ref_sections(_export(lib, p, 2 * NB).view(np.uint16),
                                      _export(lib, p, 2 * NB + 1).view(np.float32), D, C4, TIN)
        zr = hxo.patchify(z[0])[None]
        x0 = np.zeros_like(zr)
        txt16 = f16(txt)
        for code in codes:
            t0 = time.time()
            x0 = oracle_moss_rapid_step(zr, x0, txt16, code, blocks, modw, glue, vec, D=D, H=H, F=F, C4=C4, ntxt=NTXT,
                                        Ttot=TTOT, gh=GH, gw=GW)
            print(f"oracle rapid step {code} in {time.time() - t0:.1f} s", flush=True)
        ref = bn_unpatchify(x0[0], vec[7], vec[8], LAT[0], LAT[1], LAT[2])[None]
        # the same two steps without the blocks: how much of the result the blocks make
        x00 = np.zeros_like(zr)
        for code in codes:
            x00 = oracle_moss_rapid_step(zr, x00, txt16, code, [], modw, glue, vec, D=D, H=H, F=F, C4=C4, ntxt=NTXT,
                                         Ttot=TTOT, gh=GH, gw=GW)
        share = rel(x0, x00)
        r, mx = rel(got, ref), float(np.max(np.abs(got - ref)))
        print(f"rapid-moss 2 steps: x0 rel err {r:.3e}, max abs {mx:.3e}; the blocks change x0 by {share:.3f} "
              f"(relative)", flush=True)
        assert np.isfinite(got).all()
        assert share > 0.2  # the blocks make a large part of x0 (measured 1.03)
        assert r < 2.2e-3 and mx < 1.8e-2  # measured 7.4e-4, 5.8e-3
    finally:
        lib.hxa_dit_destroy(p)
