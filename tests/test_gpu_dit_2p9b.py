"""Parity of the DiT at the 2.9B-class block shape (hidden 2560, 20 heads, MLP 10240, 256 text tokens of width
1024; int8 g32, fp16 and int4 g32 weights) at 1536 image tokens against the oracle: the velocity of two chained blocks with the
caller-side glue of phone/animad.cpp:424-492 around them.

At this shape the qkv grid leaves no room for the text k / v tiles in its own launch, so the runner computes every
block's text k / v up front in one grouped launch and each block fuses its cross q with the attention; the
attention-output and MLP-down projections run fused split-K 4 into four fp16 partials. The oracle dequantises the
same int8 weights (f16(q s), gemm2.c:19-35) and computes in double with the reference block's rounding points.
Tolerance about 3x the error measured on MI355X, as the other DiT tests."""
import ctypes as C_

import numpy as np
import pytest

from oracle import hxo
from tests._helpers import f16, oracle_anima_velocity, unpack_weights

pytestmark = pytest.mark.gpu

D, H, F, C, DC, NB = 2560, 20, 10240, 256, 1024, 2
LAT = (16, 96, 64)


# weight format (0 fp16, 1 int8, 2 int4) and bounds: the fp16 and int4 forms take the same grouped text k / v launch
# (the qkv grid is the same 240 tiles); int4 runs its attention-output and MLP-down projections fused split-K 4 too
@pytest.mark.parametrize("fmt,tol", [(1, (2e-3, 9e-3)), (0, (2e-3, 9e-3)), (2, (2e-3, 9e-3))])
def test_dit_2p9b_two_blocks_velocity_vs_oracle(fmt, tol):
    from hexanima_amd import hip

    hip.init(0)
    lib = hip.lib()
    hxo.set_threads(0)
    print(f"[case] DiT fmt {fmt}, hidden 2560, 2 blocks, 1536 tokens, velocity vs oracle", flush=True)
    bd = hip.BlockDims(0, D, H, F, C, DC, 0, 1, 0, fmt, fmt, 1)
    cfg = hip.DitCfg(bd, NB, LAT[0], LAT[1], LAT[2], 256, 0)
    p = C_.c_void_p()
    hip.check(lib.hxa_dit_create(C_.byref(cfg), 91, C_.byref(p)), "dit_create")
    try:
        rng = np.random.default_rng(29)
        lat = rng.standard_normal((1,) + LAT).astype(np.float32)
        ctx = rng.standard_normal((1, C, DC)).astype(np.float32)
        hip.check(lib.hxa_dit_set_inputs(p, lat.ctypes.data, ctx.ctypes.data), "set_inputs")
        v = np.zeros_like(lat)
        hip.check(lib.hxa_dit_velocity(p, 0.75, v.ctypes.data), "velocity")

        def export(which):
            n = lib.hxa_dit_export(p, which, None, 0)
            buf = np.zeros(n, np.uint8)
            assert lib.hxa_dit_export(p, which, buf.ctypes.data, n) == n
            return buf

        layout = hip.pack_layout(0, D, F, DC, fmt, fmt)
        blocks = [unpack_weights(export(k), 0, D, F, DC, fmt, fmt, layout) for k in range(NB)]
        modws = [export(NB + k).view(np.uint16).reshape(6 * D, D) for k in range(NB)]
        g = export(2 * NB).view(np.uint16)
        C4 = 4 * LAT[0]
        glue, o = [], 0
        for (n, k) in ((D, C4), (D, 256), (2 * D, D), (C4, D)):
            glue.append(g[o:o + n * k].reshape(n, k))
            o += n * k
        ref = oracle_anima_velocity(lat, f16(ctx), 0.75, blocks, modws, glue, D=D, H=H, F=F, C4=C4, temb=256)
        r = float(np.linalg.norm(v - ref) / np.linalg.norm(ref))
        mx = float(np.max(np.abs(v - ref)))
        print(f"fmt {fmt} 2.9B-shape DiT velocity: rel err {r:.3e}, max abs {mx:.3e}", flush=True)
        assert np.isfinite(v).all()
        assert r < tol[0] and mx < tol[1]  # measured 6.2e-4 - 6.4e-4, 2.8e-3 - 3.0e-3
        if fmt == 1:
            # one low-res first step (factor 2: 384 tokens, phone/animad.cpp:429-446) through the same chain: the
            # pooled noise, the velocity on the half grid, the landing velocity, then the Euler update
            t, tn = 1.0, 0.75
            hip.check(lib.hxa_dit_step_lowres(p, t, tn, 2, 1), "step_lowres")
            got = np.zeros_like(lat)
            hip.check(lib.hxa_dit_get_latent(p, got.ctypes.data), "get_latent")
            xlow = hxo.lowres_pool(lat[0], np.zeros_like(lat[0]), 2, t)[None]
            vlow = oracle_anima_velocity(xlow, f16(ctx), t, blocks, modws, glue, D=D, H=H, F=F, C4=C4, temb=256)
            _, vl = hxo.lowres_velocity(xlow[0], vlow[0], lat[0], lat[0], 2, t, tn)
            ref2 = lat + np.float32(tn - t) * vl[None]
            d_got, d_ref = got - lat, ref2 - lat
            r2 = float(np.linalg.norm(d_got - d_ref) / np.linalg.norm(d_ref))
            mx2 = float(np.max(np.abs(got - ref2)))
            print(f"low-res step (384 tokens): rel err on delta {r2:.3e}, max abs {mx2:.3e}", flush=True)
            assert r2 < 1.2e-3 and mx2 < 1.7e-3  # measured 3.6e-4, 5.5e-4
    finally:
        lib.hxa_dit_destroy(p)
