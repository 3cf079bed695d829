"""GPU parity of the low-res first steps against the oracle: hxa_dit_step_lowres (phone/animad.cpp:392-503) and
hxa_dit_moss_step_lowres (moss/mossrun/mossrun.cpp:288-313).

The reference composition: the oracle's pooling (hxo.lowres_pool, hxo.moss_pool2), the oracle DiT at the low-res grid
(tests/_helpers: the same composition the full-resolution DiT tests use, with the grid's RoPE; MOSS with image
positions x 2), the oracle's upsampling and landing velocity (hxo.lowres_velocity, hxo.upsample2_rows), then full-res
steps. Tolerances as the full-resolution DiT tests' (about 3x the error measured on MI355X)."""
import ctypes as C

import numpy as np
import pytest

from oracle import hxo
from tests._helpers import (bn_unpatchify, delta_metrics, f16, oracle_anima_ref_velocity,
                            moss_ref_sections, oracle_moss_rapid_step, rel)
from tests.test_gpu_block import _anima_ref_weights, _export, _split, unpack_weights

pytestmark = pytest.mark.gpu

SIG = [1.0, 0.75, 0.5, 0.25, 0.0]


def _hip():
    from hexanima_amd import hip
    hip.init()
    return hip


def say(msg):
    print(f"[case] {msg}", flush=True)


def _anima(hip, batch=2, lat=32, seed=555):
    D, H, F, C_, DC, nb = 256, 2, 1024, 32, 128, 2
    bd = hip.BlockDims(0, D, H, F, C_, DC, 0, batch, 0, 0, 0, 1)
    cfg = hip.DitCfg(bd, nb, 16, lat, lat, D, 0, 1)
    p = C.c_void_p()
    hip.check(hip.lib().hxa_dit_create(C.byref(cfg), seed, C.byref(p)), "dit_create")
    return p


def test_dit_lowres_first_steps_vs_oracle():
    """Anima DiT (reference form), batch 2, latent 16 x 32 x 32 (256 tokens): two steps at factor 2 (64 tokens), then
    two full-resolution steps, against the oracle composition of animad.cpp:429-503 around the oracle DiT."""
    hip = _hip()
    say("dit low-res: 2 steps at 1/2 (64 tokens) + 2 full steps, batch 2")
    lib = hip.lib()
    p = _anima(hip)
    try:
        rng = np.random.default_rng(31)
        B, lat_hw = 2, 32
        lat = rng.standard_normal((B, 16, lat_hw, lat_hw)).astype(np.float32)
        ctx = rng.standard_normal((B, 32, 128)).astype(np.float32)
        hip.check(lib.hxa_dit_set_inputs(p, lat.ctypes.data, ctx.ctypes.data), "set_inputs")
        blocks, modws, glue = _anima_ref_weights(hip, p, 2, 256, 1024, 128, 64)
        kw = dict(D=256, H=2, F=1024, C4=64)
        ctx16 = f16(ctx)
        noise, dhat, ref = lat.copy(), np.zeros_like(lat), lat.copy()
        for i in range(4):
            t, tn = SIG[i], SIG[i + 1]
            if i < 2:
                hip.check(lib.hxa_dit_step_lowres(p, t, tn, 2, 1), "step_lowres")
                xlow = np.stack([hxo.lowres_pool(noise[b], dhat[b], 2, t) for b in range(B)])
                vlow = oracle_anima_ref_velocity(xlow, ctx16, t, blocks, modws, glue, **kw)
                v = np.empty_like(ref)
                for b in range(B):
                    dhat[b], v[b] = hxo.lowres_velocity(xlow[b], vlow[b], ref[b], noise[b], 2, t, tn)
                ref = (ref + np.float32(tn - t) * v).astype(np.float32)
            else:
                hip.check(lib.hxa_dit_step(p, t, tn, 1), "step")
                ref = ref + (tn - t) * oracle_anima_ref_velocity(ref, ctx16, t, blocks, modws, glue, **kw)
            got = np.zeros_like(lat)
            hip.check(lib.hxa_dit_get_latent(p, got.ctypes.data), "get_latent")
            r, c = delta_metrics(got, ref, lat)
            mx = float(np.max(np.abs(got - ref)))
            print(f"step {i} ({'1/2' if i < 2 else 'full'}): rel err on delta {r:.2e} cos {c:.9f} max abs {mx:.2e}",
                  flush=True)
            assert r < 4e-5 and c > 1 - 4e-5 ** 2 and mx < 9e-5  # measured 6.8e-6 - 1.3e-5, max abs 1.0e-5 - 3.0e-5
    finally:
        lib.hxa_dit_destroy(p)


def test_dit_lowres_graph_equals_eager_and_fallback_equals_full_step():
    """The low-res step replayed from its graph gives the bits of the eager one; factor 4 (16 tokens, not a multiple of
    32) runs a full-resolution step, bit-identical to hxa_dit_step."""
    hip = _hip()
    say("dit low-res: graph vs eager, factor-4 fallback")
    lib = hip.lib()
    rng = np.random.default_rng(32)
    lat = rng.standard_normal((2, 16, 32, 32)).astype(np.float32)
    ctx = rng.standard_normal((2, 32, 128)).astype(np.float32)
    outs = []
    for mode in ("graph", "eager", "fallback4", "full"):
        p = _anima(hip)
        try:
            hip.check(lib.hxa_dit_set_inputs(p, lat.ctypes.data, ctx.ctypes.data), "set_inputs")
            for i in range(3):
                if mode in ("graph", "eager"):
                    hip.check(lib.hxa_dit_step_lowres(p, SIG[i], SIG[i + 1], 2, 1 if mode == "graph" else 0), "lowres")
                elif mode == "fallback4":
                    hip.check(lib.hxa_dit_step_lowres(p, SIG[i], SIG[i + 1], 4, 1), "lowres4")
                else:
                    hip.check(lib.hxa_dit_step(p, SIG[i], SIG[i + 1], 1), "step")
            got = np.zeros_like(lat)
            hip.check(lib.hxa_dit_get_latent(p, got.ctypes.data), "get_latent")
            outs.append(got)
        finally:
            lib.hxa_dit_destroy(p)
    assert np.array_equal(outs[0], outs[1])
    assert np.array_equal(outs[2], outs[3])
    assert not np.array_equal(outs[0], outs[3])


def test_dit_moss_lowres_first_steps_vs_oracle():
    """MOSS DiT (reference form, rapid-moss sampler), batch 2, 8 x 8 token grid + 20 text tokens: two steps on the
    4 x 4 grid (noise pooled 2x2, RoPE positions x 2), then two full steps from the 2x upsampled clean estimate."""
    hip = _hip()
    say("dit moss low-res: 2 steps on the half grid + 2 full steps, batch 2")
    lib = hip.lib()
    D, H, F, ntxt, tin, nb, B = 256, 2, 512, 20, 128, 2, 2
    bd = hip.BlockDims(1, D, H, F, ntxt, 0, 0, B, 0, hip.W_Q8, hip.W_Q4, 1)
    cfg = hip.DitCfg(bd, nb, 32, 16, 16, 256, tin, 1)
    p = C.c_void_p()
    hip.check(lib.hxa_dit_create(C.byref(cfg), 777, C.byref(p)), "dit_create")
    try:
        rng = np.random.default_rng(33)
        z = rng.standard_normal((B, 32, 16, 16)).astype(np.float32)
        txt = rng.standard_normal((B, ntxt, tin)).astype(np.float32)
        hip.check(lib.hxa_dit_set_inputs(p, z.ctypes.data, txt.ctypes.data), "set_inputs")
        C4 = 128
        layout = hip.pack_layout(1, D, F, 0, hip.W_Q8, hip.W_Q4)
        blocks = [unpack_weights(_export(hip, p, k), 1, D, F, 0, hip.W_Q8, hip.W_Q4, layout) for k in range(nb)]
        modw = _export(hip, p, nb).view(np.uint16).reshape(6 * D, D)
        glue, vec = moss_ref_sections(_export(hip, p, 2 * nb).view(np.uint16),
                                      _export(hip, p, 2 * nb + 1).view(np.float32), D, C4, tin)
        codes = [0.999, 0.75, 0.5, 0.25]
        txt16 = f16(txt)
        zr = np.stack([hxo.patchify(z[b]) for b in range(B)])
        zl = np.stack([hxo.moss_pool2(zr[b], 8, 8) for b in range(B)])
        x0l = np.zeros_like(zl)
        kw = dict(D=D, H=H, F=F, C4=C4, ntxt=ntxt)
        for code in codes[:2]:
            hip.check(lib.hxa_dit_moss_step_lowres(p, code, 2.0, 1), "moss_step_lowres")
            x0l = oracle_moss_rapid_step(zl, x0l, txt16, code, blocks, modw, glue, vec, Ttot=64, gh=4, gw=4,
                                         rope_scale=2.0, **kw)
        x0 = np.stack([hxo.upsample2_rows(x0l[b], 4, 4) for b in range(B)])
        for code in codes[2:]:
            hip.check(lib.hxa_dit_moss_step(p, code, 1), "moss_step")
            x0 = oracle_moss_rapid_step(zr, x0, txt16, code, blocks, modw, glue, vec, Ttot=96, gh=8, gw=8, **kw)
        got = np.zeros_like(z)
        hip.check(lib.hxa_dit_get_latent(p, got.ctypes.data), "get_latent")
        ref = np.stack([bn_unpatchify(x0[b], vec[7], vec[8], 32, 16, 16) for b in range(B)])
        r, mx = rel(got, ref), float(np.max(np.abs(got - ref)))
        print(f"moss low-res + full output rel err {r:.2e} max abs {mx:.2e}", flush=True)
        assert r < 2e-6 and mx < 1.3e-5  # measured 6.5e-7, 4.3e-6
        assert lib.hxa_dit_step_lowres(p, 1.0, 0.5, 2, 0) == -11  # the Euler low-res step is not this form's
    finally:
        lib.hxa_dit_destroy(p)
