"""Benchmark: DiT denoise steps/s of the 2B-class fp16 DiT at 1536 tokens on one MI355X.

Workload: 28 Anima-structure blocks (hidden 2048, 16 heads x 128, MLP 8192, tanh GELU, 256 text tokens of width
1024), patch embed 64 -> 2048, final adaLN + linear 2048 -> 64, batch 1, latent 16 x 96 x 64 (1536 tokens),
random N(0, 0.02) weights, N(0, 1) latent and text. One step = one flow-matching Euler step (timestep embedding,
28 x modulation, patch embed, 28 blocks, final layer, update), replayed from a captured HIP graph with the sigma
schedule 1.0, 0.75, 0.5, 0.25 -> 0 cycled.

Prints one JSON line. `kernels` splits the block's time over its kernel families (HIP events between the block's
stages on its stream); `roofline` is for the family with the largest share -- the 192 x 128 split-K GEMM of the
o, cross-o and MLP-down projections -- timed with HIP events on the stream it is launched on, at the launch shapes
of the step. `abi_chain` runs the 28 blocks through mega_block the way megarun drives them (hxa_run, a child
process). `cpu_baseline` times the CPU oracle (a port of the reference block, built -march=native with OpenMP)
on whole blocks and one GEMM, scaled to a step.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

PEAK_FP16 = 2.5e15     # MI355X dense fp16 MFMA, FLOP/s
PEAK_HBM = 8.0e12      # bytes/s
D, H, F, C_TXT, DC, NBLK = 2048, 16, 8192, 256, 1024, 28
LAT = (16, 96, 64)
T = (LAT[1] // 2) * (LAT[2] // 2)
WFMT = 0 | 16  # fp16 weights, k-tiled: the block-pack layout of the DiT's matrices
LIN_SHAPES = ((D, 3 * D), (D, D), (D, F), (F, D))  # K x N of the block's projections (qkv, o, MLP up, MLP down)
BLOCK_FLOPS = 2 * T * D * (3 * D) + 2 * T * D * D + 2 * T * D * D + 2 * C_TXT * DC * (2 * D) + 2 * T * D * D \
    + 2 * T * D * F * 2 + 4 * T * T * D + 4 * T * C_TXT * D
STEP_FLOPS = NBLK * BLOCK_FLOPS + 2 * T * 64 * D + 2 * T * D * 64


def _event(L, hip):
    p = C.c_void_p()
    hip.check(L.hxa_event_create(C.byref(p)), "event")
    return p


def dit_ms(bd, nblk, lat_shape, ctx_shape, tin, steps, warmup, seed, wall_check=False):
    """ms per graph-replayed Euler step of a DiT (hxa_dit_*), sigma schedule 1.0, 0.75, 0.5, 0.25 -> 0 cycled.
    lat_shape = (batch, C, H, W); ctx_shape = (batch, tokens, width). The latent must stay finite."""
    from hexanima_amd import hip
    L = hip.lib()
    cfg = hip.DitCfg(bd, nblk, lat_shape[1], lat_shape[2], lat_shape[3], 256, tin)
    dit = C.c_void_p()
    hip.check(L.hxa_dit_create(C.byref(cfg), seed, C.byref(dit)), "dit_create")
    try:
        rng = np.random.default_rng(seed)
        lat = rng.standard_normal(lat_shape).astype(np.float32)
        ctx = rng.standard_normal(ctx_shape).astype(np.float32)
        hip.check(L.hxa_dit_set_inputs(dit, lat.ctypes.data, ctx.ctypes.data), "set_inputs")
        st = L.hxa_dit_stream(dit)
        sig = [1.0, 0.75, 0.5, 0.25, 0.0]
        e0, e1 = _event(L, hip), _event(L, hip)
        for i in range(warmup):
            hip.check(L.hxa_dit_step(dit, sig[i % 4], sig[i % 4 + 1], 1), "step")
        hip.check(L.hxa_stream_sync(st), "sync")
        t0 = time.perf_counter()
        hip.check(L.hxa_event_record(e0, st), "rec")
        for i in range(steps):
            hip.check(L.hxa_dit_step(dit, sig[i % 4], sig[i % 4 + 1], 1), "step")
        hip.check(L.hxa_event_record(e1, st), "rec")
        hip.check(L.hxa_stream_sync(st), "sync")
        wall = time.perf_counter() - t0
        ms = C.c_float()
        hip.check(L.hxa_event_elapsed_ms(e0, e1, C.byref(ms)), "elapsed")
        out = np.zeros_like(lat)
        hip.check(L.hxa_dit_get_latent(dit, out.ctypes.data), "latent")
        if not np.isfinite(out).all():
            raise RuntimeError("non-finite latent")
        for e in (e0, e1):
            L.hxa_event_destroy(e)
    finally:
        L.hxa_dit_destroy(dit)
    # the event interval, or the host wall clock when that is longer (nothing hidden outside the events)
    return (max(ms.value, wall * 1e3) if wall_check else ms.value) / steps


def gpu_run(steps, warmup):
    from hexanima_amd import hip
    hip.init(0)
    info = hip.device_info()
    bd = hip.BlockDims(0, D, H, F, C_TXT, DC, 0, 1, 0, hip.W_F16, hip.W_F16, 1)
    ms_step = dit_ms(bd, NBLK, (1,) + LAT, (1, C_TXT, DC), 0, steps, warmup, 2024, wall_check=True)
    return info, ms_step


def _time_launches(L, hip, fn, s, reps=20, warm=5):
    """average ms per call of fn (launches on stream s), HIP events on s"""
    e0, e1 = _event(L, hip), _event(L, hip)
    for _ in range(warm):
        fn()
    hip.check(L.hxa_event_record(e0, s), "rec")
    for _ in range(reps):
        fn()
    hip.check(L.hxa_event_record(e1, s), "rec")
    hip.check(L.hxa_stream_sync(s), "sync")
    ms = C.c_float()
    hip.check(L.hxa_event_elapsed_ms(e0, e1, C.byref(ms)), "elapsed")
    for e in (e0, e1):
        L.hxa_event_destroy(e)
    return ms.value / reps


def _rate(flops, ms):
    tf = flops / (ms * 1e-3)
    return {"us": round(ms * 1e3, 2), "tflops": round(tf / 1e12, 1), "frac_of_fp16_peak": round(tf / PEAK_FP16, 4)}


def dit_fp16_2b_batch4():
    """the 2B fp16 DiT at batch 4 (the flops scale with the batch)"""
    from hexanima_amd import hip
    bd = hip.BlockDims(0, D, H, F, C_TXT, DC, 0, 4, 0, hip.W_F16, hip.W_F16, 1)
    ms = dit_ms(bd, NBLK, (4,) + LAT, (4, C_TXT, DC), 0, 6, 1, 2026)
    return {"images_per_s": round(4000.0 / ms, 2), "ms_per_step": round(ms, 3),
            "step_tflops": round(4 * STEP_FLOPS / (ms * 1e-3) / 1e12, 1),
            "config": "28 blocks, hidden 2048, batch 4 x 1536 tokens, fp16"}


def dit_q8_2p9b():
    """the 2.9B-class DiT with int8 group-32 block linears"""
    from hexanima_amd import hip
    Dq, Hq, Fq = 2560, 20, 10240
    bd = hip.BlockDims(0, Dq, Hq, Fq, C_TXT, DC, 0, 1, 0, hip.W_Q8, hip.W_Q8, 1)
    ms = dit_ms(bd, NBLK, (1,) + LAT, (1, C_TXT, DC), 0, 10, 2, 2025)
    blk = 2 * T * Dq * (3 * Dq) + 3 * 2 * T * Dq * Dq + 2 * C_TXT * DC * 2 * Dq + 2 * 2 * T * Dq * Fq \
        + 4 * T * T * Dq + 4 * T * C_TXT * Dq
    return {"steps_per_s": round(1000.0 / ms, 3), "ms_per_step": round(ms, 4),
            "step_tflops": round(NBLK * blk / (ms * 1e-3) / 1e12, 1),
            "config": "28 blocks, hidden 2560, 20 heads, MLP 10240, int8 g32 block linears, "
                      "1536 image + 256 text tokens"}


def dit_moss():
    """the MOSS-class DiT: 36 blocks, hidden 3072, 24 heads, MLP 12288 SiTU-gated, int8 attention / int4 MLP
    weights, joint attention over 6144 image + 512 text tokens of width 4096 projected to 3072 (latent 32 x 128 x
    192 -> 64 x 96 patch grid)"""
    from hexanima_amd import hip
    Dm, Hm, Fm, NBm, NTXT, TIN = 3072, 24, 12288, 36, 512, 4096
    bd = hip.BlockDims(1, Dm, Hm, Fm, NTXT, 0, 0, 1, 0, hip.W_Q8, hip.W_Q4, 1)
    ms = dit_ms(bd, NBm, (1, 32, 128, 192), (1, NTXT, TIN), TIN, 3, 1, 2027)
    Tm = 6144 + NTXT
    blk = 2 * Tm * Dm * 4 * Dm + 2 * Tm * Dm * 2 * Fm + 2 * Tm * Fm * Dm + 4 * Tm * Tm * Dm
    return {"steps_per_s": round(1000.0 / ms, 3), "ms_per_step": round(ms, 2),
            "step_tflops": round(NBm * blk / (ms * 1e-3) / 1e12, 1),
            "step_frac_of_fp16_peak": round(NBm * blk / (ms * 1e-3) / PEAK_FP16, 4),
            "config": "36 blocks, hidden 3072, 24 heads, MLP 12288 SiTU, int8 attention / int4 MLP "
                      "g32, joint attention 6144 image + 512 text tokens"}


EXTRA_DITS = {"fp16_2b_dit_batch4": dit_fp16_2b_batch4, "q8_2p9b_dit": dit_q8_2p9b, "moss_5b_dit": dit_moss}


def extra_dits():
    """The other DiT workloads, each as ms per graph-replayed Euler step."""
    return {k: f() for k, f in EXTRA_DITS.items()}


def microbench():
    """Kernel-level figures on the benchmark shapes (HIP events, inputs resident in HBM):
    - W8A16 / W4A16 linears at M = 1536 (K x N = 2048 x 6144, 2048 x 2048, 2048 x 8192, 8192 x 2048; int8 uniform in
      [-127, 127] / int4 uniform in [-8, 7], group-32 fp16 scales 0.02/127, pack layout), beside fp16 weights, through
      hxa_linear (one launch storing fp16, or for the long-K shapes K slices into fp32 partials and their sum; the
      one-launch time is given beside it there); and the N <= K shapes in the form the block runs them with int8 /
      int4 weights (fused, split-K 4 into fp16 partials);
    - attention: the 2B block's self (1536 x 1536, 16 heads) and cross (1536 x 256) attention, and the MOSS-class
      joint attention (6656 x 6656, 24 heads);
    - one 2B fp16 block (hxa_block_run, 1536 tokens), the block latency."""
    from hexanima_amd import hip
    L = hip.lib()
    s = C.c_void_p()
    hip.check(L.hxa_stream_create(C.byref(s)), "stream")
    res = {"linear_m1536": {}, "linear_m1536_2p9b": {}, "attention": {}}
    M = T
    A = hip.DeviceArray((M, 10240), np.float16)
    hip.check(L.hxa_fill_normal(A.ptr, 1, M * 10240, 21, 0.0, 1.0, s), "fill")
    Wb = hip.DeviceArray((10240 * 2560 * 2,), np.uint8)
    Sb = hip.DeviceArray((320 * 10240,), np.float16)
    O = hip.DeviceArray((M, 10240), np.float16)
    WS = hip.DeviceArray((4 * M * 2560 * 4,), np.uint8)  # hxa_linear's fp32 slices (split shapes have N <= 2560)
    hip.check(L.hxa_fill_const(Sb.ptr, 1, 320 * 10240, 0.02 / 127, s), "fill")
    # the 2B block's projections in each format, and the 2.9B-class block's (hidden 2560, MLP 10240) in fp16 / int8
    for key, shapes, fmts in (("linear_m1536", ((2048, 6144), (2048, 2048), (2048, 8192), (8192, 2048)),
                               (("fp16", hip.W_F16), ("q8", hip.W_Q8), ("q4", hip.W_Q4))),
                              ("linear_m1536_2p9b", ((2560, 7680), (2560, 2560), (2560, 10240), (10240, 2560)),
                               (("fp16", hip.W_F16), ("q8", hip.W_Q8), ("q4", hip.W_Q4)))):
        for name, fmt in fmts:
            row = {}
            for K, N in shapes:
                assert N * K <= 10240 * 2560 and K <= 10240 and N <= 10240
                if fmt == hip.W_F16:
                    hip.check(L.hxa_fill_normal(Wb.ptr, 1, N * K, 22, 0.0, 0.02, s), "fill")
                elif fmt == hip.W_Q8:
                    hip.check(L.hxa_fill_uniform_int(Wb.ptr, 8, N * K, 23, -127, 127, s), "fill")
                else:
                    hip.check(L.hxa_fill_uniform_int(Wb.ptr, 4, N * K // 2, 24, -8, 7, s), "fill")
                sp = None if fmt == hip.W_F16 else Sb.ptr

                def run(K=K, N=N, fmt=fmt, sp=sp):
                    hip.check(L.hxa_gemm(A.ptr, K, M, fmt | hip.W_KTILED, Wb.ptr, sp, None, N, K, 1, hip.EPI_STORE, O.ptr,
                                         N, 0, None, 0, None, None, 0, 0, s), "gemm")

                def lin(K=K, N=N, fmt=fmt, sp=sp):
                    hip.check(L.hxa_linear(A.ptr, K, M, fmt | hip.W_KTILED, Wb.ptr, sp, None, N, K, O.ptr, N, WS.ptr,
                                           WS.nbytes, s), "linear")
                nsplit = L.hxa_linear_split_k(M, N, K, fmt)
                assert L.hxa_linear_ws_bytes(M, N, K, fmt) <= WS.nbytes
                r = _rate(2.0 * M * N * K, _time_launches(L, hip, lin, s))
                r["split_k"] = nsplit
                if nsplit > 1:
                    r["one_launch_us"] = round(1e3 * _time_launches(L, hip, run, s), 2)
                row[f"{K}x{N}"] = r
            res[key][name] = row
    # the N <= K projections as the block runs them with int8 / int4 weights at 1536 tokens: fused, split-K 4 into
    # four fp16 partials (the next norm adds them); fp16 in the same form for comparison
    res["linear_m1536_splitk4"] = {}
    for name, fmt, shapes in (("fp16", hip.W_F16, ((2048, 2048), (8192, 2048), (2560, 2560), (10240, 2560))),
                              ("q8", hip.W_Q8, ((2048, 2048), (8192, 2048), (2560, 2560), (10240, 2560))),
                              ("q4", hip.W_Q4, ((2048, 2048), (8192, 2048)))):
        row = {}
        for K, N in shapes:
            assert 4 * N <= 10240
            if fmt == hip.W_F16:
                hip.check(L.hxa_fill_normal(Wb.ptr, 1, N * K, 22, 0.0, 0.02, s), "fill")
            elif fmt == hip.W_Q8:
                hip.check(L.hxa_fill_uniform_int(Wb.ptr, 8, N * K, 23, -127, 127, s), "fill")
            else:
                hip.check(L.hxa_fill_uniform_int(Wb.ptr, 4, N * K // 2, 24, -8, 7, s), "fill")
            sp = None if fmt == hip.W_F16 else Sb.ptr

            def run4(K=K, N=N, fmt=fmt, sp=sp):
                hip.check(L.hxa_gemm(A.ptr, K, M, fmt | hip.W_KTILED, Wb.ptr, sp, None, N, K, 4, hip.EPI_PARTIAL, O.ptr,
                                     N, M * N, None, 0, None, None, 0, 0, s), "gemm")
            row[f"{K}x{N}"] = _rate(2.0 * M * N * K, _time_launches(L, hip, run4, s))
        res["linear_m1536_splitk4"][name] = row
    # attention (q, k, v^T resident; random fp16)
    for name, Tq, NKV, Hh in (("self_1536x1536_h16", T, T, H), ("cross_1536x256_h16", T, C_TXT, H),
                              ("joint_6656x6656_h24", 6656, 6656, 24)):
        Dd = Hh * 128
        q = hip.DeviceArray((Tq, Dd), np.float16)
        k = hip.DeviceArray((NKV, Dd), np.float16)
        vt = hip.DeviceArray((Dd, NKV), np.float16)
        o = hip.DeviceArray((Tq, Dd), np.float16)
        for i, t in enumerate((q, k, vt)):
            hip.check(L.hxa_fill_normal(t.ptr, 1, t.nbytes // 2, 30 + i, 0.0, 1.0, s), "fill")

        def att(q=q, k=k, vt=vt, o=o, Tq=Tq, NKV=NKV, Dd=Dd, Hh=Hh):
            hip.check(L.hxa_attention(q.ptr, Dd, k.ptr, Dd, vt.ptr, NKV, o.ptr, Dd, Tq, NKV, NKV, Hh, 1, 0, 0, 0, 0, s),
                      "attention")
        res["attention"][name] = _rate(4.0 * Tq * NKV * Dd, _time_launches(L, hip, att, s))
        del q, k, vt, o
    # one 2B fp16 block
    blk, _keep = _block_setup(L, hip, s)
    res["block_2b_fp16_1536tok"] = _rate(BLOCK_FLOPS, _time_launches(L, hip, blk, s, reps=10, warm=2))
    hip.check(L.hxa_stream_sync(s), "sync")
    L.hxa_stream_destroy(s)
    return res


def _block_setup(L, hip, s):
    """The 2B fp16 block on resident synthetic data (weights N(0, 0.02), x N(0, 1), text N(0, 1), modulation
    N(0, 0.02), identity RoPE); returns blk(stage_us=None), one hxa_block_run on stream s, and the buffers it uses."""
    bd = hip.BlockDims(0, D, H, F, C_TXT, DC, T, 1, T, hip.W_F16, hip.W_F16, 1)
    total, mats, voff = hip.pack_layout(0, D, F, DC, hip.W_F16, hip.W_F16)
    pack = hip.DeviceArray((total,), np.uint8)
    for i, ((n, kk), (wo, _)) in enumerate(zip(hip.pack_shapes(0, D, F, DC), mats)):
        hip.check(L.hxa_fill_normal(C.c_void_p(pack.ptr + wo), 1, n * kk, 40 + i, 0.0, 0.02, s), "fill")
    gain = np.concatenate([np.full(128, 128 ** -0.5), np.ones(128), np.full(128, 128 ** -0.5), np.ones(128)]).astype(np.float32)
    hip.check(L.hxa_h2d(C.c_void_p(pack.ptr + voff), gain.ctypes.data, 4 * 512), "gain")
    x = hip.DeviceArray((T, D), np.float32)
    ctx = hip.DeviceArray((C_TXT, DC), np.float16)
    mod = hip.DeviceArray((9, D), np.float32)
    hip.check(L.hxa_fill_normal(x.ptr, 0, T * D, 50, 0.0, 1.0, s), "fill")
    hip.check(L.hxa_fill_normal(ctx.ptr, 1, C_TXT * DC, 51, 0.0, 1.0, s), "fill")
    hip.check(L.hxa_fill_normal(mod.ptr, 0, 9 * D, 52, 0.0, 0.02, s), "fill")
    cos, sin = hip.DeviceArray((T, 64), np.float32), hip.DeviceArray((T, 64), np.float32)
    hip.check(L.hxa_fill_const(cos.ptr, 0, T * 64, 1.0, s), "fill")
    hip.check(L.hxa_fill_const(sin.ptr, 0, T * 64, 0.0, s), "fill")
    ws = hip.block_ws(bd)

    def blk(stage_us=None):
        hip.check(L.hxa_block_run(C.byref(bd), pack.ptr, x.ptr, ctx.ptr, mod.ptr, cos.ptr, sin.ptr, ws.ptr, 0, stage_us,
                                  24 if stage_us is not None else 0, s), "block")
    return blk, (bd, pack, x, ctx, mod, cos, sin, ws)


# The Anima block's 13 stages (blk.c:136 TICK order) and the kernel family each one launches.
# At 1536 tokens the text k / v projection runs in the qkv launch (its tiles on the CUs the qkv grid leaves idle)
# and the cross q projection is fused with the cross attention, so stages 2, 7 and 8 launch nothing.
STAGES = ("LN-mod self", "qkv + head RMSNorm + RoPE (+ text k/v tiles)", "(RoPE: fused)", "self attention",
          "o projection", "LN-mod cross", "cross q + RMSNorm + cross attention (fused)", "(RMSNorm: fused)",
          "(cross attention: fused)", "cross-o projection", "LN-mod MLP", "MLP up + GELU", "MLP down")
FAMILIES = {  # family -> the stages whose launches it is
    "gemm_splitk": (4, 9, 12),
    "gemm_pp_mlp_up": (11,),
    "gemm_pp_qkv_headnorm": (1,),
    "attention": (3,),
    "gemm_xattn_cross": (6,),
    "normrow": (0, 5, 10),
}


def _kname(pk):
    return (f"{'gemm_pp_kernel' if pk['waves'] == 9 else 'gemm_kernel'} {pk['bm']}x{pk['bn']}"
            f" ({8 if pk['waves'] == 9 else pk['waves']} waves)")


def family_launchers(L, hip, s):
    """The launches of the GEMM and attention families at their in-step shapes (batch 1, 1536 tokens, 256 text
    tokens), on resident synthetic fp16 data: family -> (fn launching the family's launches of one block once,
    launches, algorithmic FLOP of those launches, algorithmic HBM bytes of those launches (operands read once,
    results written once), kernel name), plus the buffers to keep alive."""
    keep = []

    def arr(shape, seed, std=1.0):
        a = hip.DeviceArray(shape, np.float16)
        hip.check(L.hxa_fill_normal(a.ptr, 1, int(np.prod(shape)), seed, 0.0, std, s), "fill")
        keep.append(a)
        return a
    h, mid, o = arr((T, D), 61), arr((T, F), 62), arr((T, D), 63)
    Wo, Wco, W1, W2, Wqkv = arr((D, D), 64, 0.02), arr((D, D), 65, 0.02), arr((F, D), 66, 0.02), arr((D, F), 67, 0.02), \
        arr((3 * D, D), 68, 0.02)
    part, up, qk, vt = arr((2, T, D), 69), arr((T, F), 70), arr((T, 2 * D), 71), arr((D, T), 72)
    k, ck, cvt = arr((T, D), 73), arr((C_TXT, D), 74), arr((D, C_TXT), 75)
    gain = hip.DeviceArray((512,), np.float32)
    cs, sn = hip.DeviceArray((T, 64), np.float32), hip.DeviceArray((T, 64), np.float32)
    keep += [gain, cs, sn]
    hip.check(L.hxa_fill_const(gain.ptr, 0, 512, 128 ** -0.5, s), "fill")
    hip.check(L.hxa_fill_const(cs.ptr, 0, T * 64, 1.0, s), "fill")
    hip.check(L.hxa_fill_const(sn.ptr, 0, T * 64, 0.0, s), "fill")
    P = hip.EPI_PARTIAL

    def splitk(hook=None):  # o, cross-o (K = D) and MLP down (K = F): two fp16 K-half partials each
        for i, (A, lda, W, K) in enumerate(((o, D, Wo, D), (o, D, Wco, D), (mid, F, W2, F))):
            if hook:
                hook(i)
            hip.check(L.hxa_gemm(A.ptr, lda, T, WFMT, W.ptr, None, None, D, K, 2, P, part.ptr, D, T * D, None, 0, None,
                                 None, 0, 0, s), "gemm")

    def mlp_up(hook=None):
        if hook:
            hook(0)
        hip.check(L.hxa_gemm(h.ptr, D, T, WFMT, W1.ptr, None, None, F, D, 1, hip.EPI_GELU_TANH, up.ptr, F, 0, None, 0,
                             None, None, 0, 0, s), "gemm")

    def qkv(hook=None):
        if hook:
            hook(0)
        hip.check(L.hxa_gemm_headnorm(h.ptr, D, T, WFMT, Wqkv.ptr, None, None, 3 * D, D, qk.ptr, 2 * D, vt.ptr, T, 2 * D,
                                      2 * D, gain.ptr, gain.ptr, D, cs.ptr, sn.ptr, T, s), "gemm_headnorm")

    def attention(hook=None):
        if hook:
            hook(0)
        hip.check(L.hxa_attention(qk.ptr, 2 * D, k.ptr, D, vt.ptr, T, o.ptr, D, T, T, T, H, 1, 0, 0, 0, 0, s), "attn")

    def xattn(hook=None):
        if hook:
            hook(0)
        hip.check(L.hxa_cross_attention_fused(h.ptr, D, T, T, WFMT, Wco.ptr, D, D, gain.ptr, ck.ptr, D, cvt.ptr, C_TXT,
                                              C_TXT, C_TXT, 0, 0, o.ptr, D, s), "cross_attention_fused")
    def linears(fmt):  # the block's four projection shapes at 1536 rows, plain store, fp16 / int8 / int4 weights
        wts = []

        def run(hook=None):
            if not wts:  # weights made on the first call
                Wq, Sq = hip.DeviceArray((F * D * 2,), np.uint8), hip.DeviceArray((F // 32 * D,), np.float16)
                wts.extend([Wq, Sq])
                if fmt == 0:
                    hip.check(L.hxa_fill_normal(Wq.ptr, 1, F * D, 81, 0.0, 0.02, s), "fill")
                else:
                    lo, hi = (-127, 127) if fmt == 1 else (-8, 7)
                    hip.check(L.hxa_fill_uniform_int(Wq.ptr, 8 if fmt == 1 else 4, F * D // (1 if fmt == 1 else 2), 82,
                                                     lo, hi, s), "fill")
                    hip.check(L.hxa_fill_const(Sq.ptr, 1, F // 32 * D, 0.02 / hi, s), "fill")
            Wq, Sq = wts
            for i, (K, N) in enumerate(LIN_SHAPES):
                if hook:
                    hook(i)
                hip.check(L.hxa_gemm(mid.ptr, K, T, fmt | 16, Wq.ptr, None if fmt == 0 else Sq.ptr, None, N, K, 1,
                                     hip.EPI_STORE, up.ptr, N, 0, None, 0, None, None, 0, 0, s), "gemm")
        return run
    f16 = 2
    lin_flops = sum(2 * T * K * N for K, N in LIN_SHAPES)
    lin_bytes = {f: sum(T * K * 2 + N * K * wb + T * N * 2 + (K // 32 * N * 2 if f else 0) for K, N in LIN_SHAPES)
                 for f, wb in ((0, 2), (1, 1), (2, 0.5))}
    fam = {
        "gemm_splitk": (splitk, 3, 2 * T * D * D * 2 + 2 * T * F * D,
                        f16 * (2 * (T * D + D * D + 2 * T * D) + (T * F + D * F + 2 * T * D)),
                        _kname(hip.gemm_pick(T, D, F, WFMT, 2, P)) + " split-K 2, fp16 partials"),
        "gemm_pp_mlp_up": (mlp_up, 1, 2 * T * D * F, f16 * (T * D + F * D + T * F),
                           _kname(hip.gemm_pick(T, F, D, WFMT, 1, hip.EPI_GELU_TANH)) + ", GELU epilogue"),
        "gemm_pp_qkv_headnorm": (qkv, 1, 2 * T * D * 3 * D, f16 * (T * D + 3 * D * D + 3 * T * D),
                                 _kname(hip.gemm_pick(T, 3 * D, D, WFMT, 1, 0, 2 * D)) + ", head RMSNorm + RoPE epilogue"
                                 " (timed without the text k/v tiles the step's launch adds)"),
        "attention": (attention, 1, 4 * T * T * D, f16 * (4 * T * D), "attn_kernel (128-query workgroups)"),
        "gemm_xattn_cross": (xattn, 1, 2 * T * D * D + 4 * T * C_TXT * D, f16 * (T * D + D * D + 2 * C_TXT * D + T * D),
                             "gemm_xattn_kernel 128x128 (4 waves): cross q + head RMSNorm, attention over the text keys"),
    }
    for f, nm in ((0, "f16"), (1, "q8"), (2, "q4")):
        picks = ", ".join(_kname(hip.gemm_pick(T, N, K, f, 1, 0)) for K, N in LIN_SHAPES)
        fam["linears_" + nm] = (linears(f), len(LIN_SHAPES), lin_flops, lin_bytes[f],
                                f"K x N {', '.join(f'{K}x{N}' for K, N in LIN_SHAPES)}: {picks}")
    # the MLP-down shape (K 8192, N 2048, 1536 rows) through hxa_linear: K slices into fp32 partials, then their sum
    lws = hip.DeviceArray((4 * T * D * 4,), np.uint8)
    keep.append(lws)
    for f, nm in ((0, "f16"), (1, "q8"), (2, "q4")):
        K, N, wb = F, D, (2.0, 1.0, 0.5)[f]
        Wq, Sq = hip.DeviceArray((N * K * 2,), np.uint8), hip.DeviceArray((K // 32 * N,), np.float16)
        keep += [Wq, Sq]
        if f == 0:
            hip.check(L.hxa_fill_normal(Wq.ptr, 1, N * K, 83, 0.0, 0.02, s), "fill")
        else:
            lo, hi = (-127, 127) if f == 1 else (-8, 7)
            hip.check(L.hxa_fill_uniform_int(Wq.ptr, 8 if f == 1 else 4, N * K // (1 if f == 1 else 2), 84, lo, hi, s),
                      "fill")
            hip.check(L.hxa_fill_const(Sq.ptr, 1, K // 32 * N, 0.02 / hi, s), "fill")
        S = L.hxa_linear_split_k(T, N, K, f)
        assert 1 < S <= 4 and L.hxa_linear_ws_bytes(T, N, K, f) <= lws.nbytes

        def lin_run(hook=None, f=f, Wq=Wq, Sq=Sq, K=K, N=N):
            hip.check(L.hxa_linear(mid.ptr, K, T, f | 16, Wq.ptr, None if f == 0 else Sq.ptr, None, N, K, up.ptr, N,
                                   lws.ptr, lws.nbytes, s), "linear")
        fam["linear_split_" + nm] = (
            lin_run, 2, 2 * T * K * N, T * K * 2 + N * K * wb + (K // 32 * N * 2 if f else 0) + T * N * 2,
            f"hxa_linear K x N {K}x{N}: {_kname(hip.gemm_pick(T, N, K, f, S, hip.EPI_PARTIAL_F32))} split-K {S} "
            f"(fp32 partials) + sum_partials_kernel")
    return fam, keep


def kernel_breakdown(L, hip, reps=10):
    """Per-stage microseconds of the 2B fp16 block (HIP events between its stages, `reps` blocks after 2 warm-up),
    grouped into kernel families, each family's launches timed alone at the step's shapes, and the roofline of the
    family with the largest share of the block."""
    s = C.c_void_p()
    hip.check(L.hxa_stream_create(C.byref(s)), "stream")
    blk, keep = _block_setup(L, hip, s)
    acc = np.zeros(len(STAGES))
    st = (C.c_int * 24)()
    for r in range(reps + 2):
        blk(st)
        if r >= 2:
            acc += np.array(st[:len(STAGES)], dtype=np.float64)
    us = acc / reps
    block_us = float(us.sum())
    fam, keep2 = family_launchers(L, hip, s)
    table = {}
    for name, stages in FAMILIES.items():
        row = {"stages": [STAGES[i] for i in stages], "block_us": round(float(us[list(stages)].sum()), 1),
               "share_of_block": round(float(us[list(stages)].sum()) / block_us, 4)}
        if name in fam:
            fn, n, flops, nbytes, kname = fam[name]
            ms = _time_launches(L, hip, fn, s, reps=30, warm=5)
            row.update({"kernel": kname, "launches": n, "avg_launch_us": round(ms * 1e3 / n, 2),
                        "gflop_per_launch": round(flops / n / 1e9, 3), "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
                        "frac_of_fp16_peak": round(flops / (ms * 1e-3) / PEAK_FP16, 4),
                        "alg_mb_per_launch": round(nbytes / n / 1e6, 2)})
        table[name] = row
    dom = max(table, key=lambda k: table[k]["block_us"] if k in fam else -1.0)
    fn, n, flops, nbytes, kname = fam[dom]
    ms = _time_launches(L, hip, fn, s, reps=50, warm=5)
    clocks = _family_clocks(L, hip, fn, n, s, kind=1 if dom == "attention" else 0)
    hip.check(L.hxa_stream_sync(s), "sync")
    L.hxa_stream_destroy(s)
    del keep, keep2
    traffic = None
    tpath = os.path.join(ROOT, "profiles", f"traffic_{dom}_1536tok.txt")
    if os.path.exists(tpath):  # rocprofv3 FETCH_SIZE + WRITE_SIZE per launch, copy-calibrated (see that file)
        for line in open(tpath):
            if line.startswith("hbm_bytes_per_launch:"):
                traffic = int(line.split(":")[1])
    tf = flops / (ms * 1e-3)
    ghz = float(np.mean([c["ghz"] for c in clocks]))
    peak_clk = CLK_FLOPS_PER_CYCLE * ghz * 1e9
    roof = {"kernel": f"{kname}: {dom} ({', '.join(table[dom]['stages'])}), {n} launches per block",
            "bound": "mfma", "achieved": round(tf / 1e12, 1), "peak": PEAK_FP16 / 1e12, "unit": "TFLOP/s",
            "frac": round(tf / PEAK_FP16, 4), "traffic": traffic, "avg_launch_us": round(ms * 1e3 / n, 2),
            "gflop_per_launch": round(flops / n / 1e9, 3), "alg_bytes_per_launch": int(nbytes // n),
            "share_of_block": table[dom]["share_of_block"],
            "clock_ghz": round(ghz, 3), "peak_at_clock": round(peak_clk / 1e12, 1),
            "frac_at_clock": round(tf / peak_clk, 4), "clock_by_launch": clocks}
    return {"block_us_staged": round(block_us, 1), "families": table}, roof


CLK_FLOPS_PER_CYCLE = 256 * 4 * 1024  # 256 CUs x 4 SIMDs x 1024 fp16 MFMA flops per SIMD per cycle (2.5 PF at 2.4 GHz)


def _records(L, hip, rec, nwg):
    """(clock GHz, main-loop cycles) per workgroup from a shader-clock record (hxa_clock_record)"""
    buf = np.zeros(nwg * 4, np.uint64)
    hip.check(L.hxa_d2h(buf.ctypes.data, rec.ptr, buf.nbytes), "d2h")
    b = buf.reshape(nwg, 4).astype(np.float64)
    ok = b[:, 3] > b[:, 1]
    cyc, real = b[ok, 2] - b[ok, 0], b[ok, 3] - b[ok, 1]
    return cyc / real * 0.1, cyc, int(ok.sum())


def _family_clocks(L, hip, fn, n, s, kind=0, reps=50, maxwg=4096):
    """The shader clock of each launch of a kernel family (kind 0: GEMM, 1: attention), run back to back `reps` times
    with a clock record per launch (the records keep the last repetition): per launch the mean clock over its
    workgroups and its main-loop cycles."""
    recs = [hip.DeviceArray((maxwg * 4,), np.uint64) for _ in range(n)]
    for r in recs:
        hip.check(L.hxa_memset(r.ptr, 0, r.nbytes), "memset")
    for _ in range(reps):
        fn(lambda i: hip.check(L.hxa_clock_record(kind, recs[i].ptr, maxwg), "clock_record"))
    hip.check(L.hxa_clock_record(kind, None, 0), "clock_record")
    hip.check(L.hxa_stream_sync(s), "sync")
    out = []
    for r in recs:
        ghz, cyc, nwg = _records(L, hip, r, maxwg)
        out.append({"ghz": round(float(ghz.mean()), 3), "loop_cycles": round(float(cyc.mean())), "workgroups": nwg})
    return out


def clock_probe():
    """Shader clock and main-loop cycles of the MLP-up GEMM (1536 x 8192, K 2048, fp16 k-tiled weights, the tile
    hxa_gemm picks) launched 40 times back to back: with N(0, 1) activations and N(0, 0.02) weights, with both zero,
    and on one workgroup (M x N = one tile) with random data; then the clock of the 2B DiT step's GEMM and attention
    launches (the last launch of each, graph-replayed steps). One JSON line."""
    from hexanima_amd import hip
    hip.init(0)
    L = hip.lib()
    s = C.c_void_p()
    hip.check(L.hxa_stream_create(C.byref(s)), "stream")
    K, N = D, F
    pk = hip.gemm_pick(T, N, K, WFMT, 1, 0)
    bm, bn = pk["bm"], pk["bn"]
    A = hip.DeviceArray((T, K), np.float16)
    W = hip.DeviceArray((N, K), np.float16)
    O = hip.DeviceArray((T, N), np.float16)
    rec = hip.DeviceArray((4096 * 4,), np.uint64)
    res = {"gemm": f"{T}x{N}x{K} fp16, {_kname(pk)}", "cases": []}
    for name, M_, N_, astd, wstd in (("full chip, random data", T, N, 1.0, 0.02), ("full chip, zero data", T, N, 0.0, 0.0),
                                     ("one workgroup, random data", bm, bn, 1.0, 0.02)):
        hip.check(L.hxa_fill_normal(A.ptr, 1, T * K, 81, 0.0, astd, s), "fill")
        hip.check(L.hxa_fill_normal(W.ptr, 1, N * K, 82, 0.0, wstd, s), "fill")
        hip.check(L.hxa_memset(rec.ptr, 0, rec.nbytes), "memset")

        def run(M_=M_, N_=N_):  # the tile picked for the full shape, also on one workgroup
            hip.check(L.hxa_gemm_tile(A.ptr, K, M_, WFMT, W.ptr, None, None, N_, K, 1, 0, O.ptr, N_, 0, None, 0, None, bm, bn,
                                      pk["waves"], s), "gemm")
        ms = _time_launches(L, hip, run, s, reps=40, warm=10)
        hip.check(L.hxa_clock_record(0, rec.ptr, 4096), "clock_record")
        for _ in range(40):
            run()
        hip.check(L.hxa_clock_record(0, None, 0), "clock_record")
        hip.check(L.hxa_stream_sync(s), "sync")
        ghz, cyc, nwg = _records(L, hip, rec, 4096)
        flops = 2.0 * M_ * N_ * K
        res["cases"].append({"case": name, "launch_us": round(ms * 1e3, 2), "workgroups": nwg,
                             "clock_ghz": round(float(ghz.mean()), 3), "clock_min_max": [round(float(ghz.min()), 3),
                                                                                        round(float(ghz.max()), 3)],
                             "loop_cycles": round(float(cyc.mean())), "tflops": round(flops / (ms * 1e-3) / 1e12, 1)})
    del A, W, O
    # the DiT step: records on while the graph is captured (the step's launches carry them), last launch kept
    recs = [hip.DeviceArray((4096 * 4,), np.uint64) for _ in range(2)]
    for k, r in enumerate(recs):
        hip.check(L.hxa_memset(r.ptr, 0, r.nbytes), "memset")
        hip.check(L.hxa_clock_record(k, r.ptr, 4096), "clock_record")
    bd = hip.BlockDims(0, D, H, F, C_TXT, DC, 0, 1, 0, hip.W_F16, hip.W_F16, 1)
    ms = dit_ms(bd, NBLK, (1,) + LAT, (1, C_TXT, DC), 0, 20, 3, 2024)
    for k in range(2):
        hip.check(L.hxa_clock_record(k, None, 0), "clock_record")
    step = {"ms_per_step": round(ms, 3)}
    for k, name in enumerate(("last_gemm", "last_attention")):
        ghz, cyc, nwg = _records(L, hip, recs[k], 4096)
        step[name] = {"clock_ghz": round(float(ghz.mean()), 3), "workgroups": nwg}
    res["dit_step_2b"] = step
    L.hxa_stream_destroy(s)
    print(json.dumps(res), flush=True)


def kernel_probe(reps, family):
    """Launches only one kernel family's in-step launches (`reps` times) and a 256 MiB device-to-device copy (3 times,
    the byte-count calibration of the FETCH_SIZE / WRITE_SIZE counters), for `rocprofv3 --pmc` passes."""
    from hexanima_amd import hip
    hip.init(0)
    L = hip.lib()
    s = C.c_void_p()
    hip.check(L.hxa_stream_create(C.byref(s)), "stream")
    fam, keep = family_launchers(L, hip, s)
    fn, n, flops, nbytes, kname = fam[family]
    for _ in range(reps):
        fn()
    # the same launches again between two HIP events (bench.py's own timing), so a kernel trace of this command holds
    # both: its mean over the second `reps` groups and this average describe the same launches
    ev_us = _time_launches(L, hip, fn, s, reps=reps, warm=0) * 1e3 / n
    nb = 256 << 20
    src = hip.DeviceArray((nb,), np.uint8)
    dst = hip.DeviceArray((nb,), np.uint8)
    hip.check(L.hxa_stream_sync(s), "sync")
    hip.check(L.hxa_memset(src.ptr, 1, nb), "memset")
    for _ in range(3):
        hip.check(L.hxa_d2d(dst.ptr, src.ptr, nb), "copy")
    hip.check(L.hxa_stream_sync(s), "sync")
    print(f"kernel probe: {reps} x {family} ({n} launches, {kname}, {nbytes / n:.0f} algorithmic bytes per launch),"
          f" then {reps} x again between HIP events: {ev_us:.2f} us per launch; 3 x copy {nb} B", flush=True)


BLK_W_END, BLK_GAIN, BLK_MODW, BLK_TOTAL = 125829120, 125829120, 125833216, 138416128  # blk_wlayout.h:3-20


def abi_chain(runs=3):
    """The 28 blocks through the reference ABI the way megarun drives them (megarun.cpp:132-195): hxa_run, the
    megarun protocol on mega_open / mega_block, as a child process holding 28 registered fp16 blkNN.bin buffers
    (one synthetic file: N(0, 0.02) fp16 weights and modulation weights, q/k gains 1/sqrt(128)), 1536 tokens
    (48 x 32 grid) and 512 context tokens. Per `run`: GPU modulation of the 28 blocks, then 28 mega_block calls,
    FIRST on the first (x uploaded) and REL on the last (x downloaded). One warm-up run converts the weights."""
    import subprocess
    import tempfile
    exe = os.path.join(ROOT, "hexanima_amd", "hxa_run")
    if not os.access(exe, os.X_OK):
        raise RuntimeError(f"{exe} is not built")
    rng = np.random.default_rng(77)
    buf = np.zeros(BLK_TOTAL, np.uint8)
    buf[:BLK_W_END] = (rng.standard_normal(BLK_W_END // 2, dtype=np.float32) * 0.02).astype(np.float16).view(np.uint8)
    gain = np.concatenate([np.full(128, 128 ** -0.5), np.ones(128), np.full(128, 128 ** -0.5), np.ones(128)])
    buf[BLK_GAIN:BLK_GAIN + 2048] = gain.astype(np.float32).view(np.uint8)
    buf[BLK_MODW:] = (rng.standard_normal((BLK_TOTAL - BLK_MODW) // 2, dtype=np.float32) * 0.02).astype(np.float16).view(np.uint8)
    gh, gw, nctx = 48, 32, 512
    with tempfile.TemporaryDirectory() as td:
        buf.tofile(os.path.join(td, "blk00.bin"))
        del buf
        for i in range(1, NBLK):
            os.symlink("blk00.bin", os.path.join(td, f"blk{i:02d}.bin"))
        rng.standard_normal((D, gh * gw), dtype=np.float32).tofile(os.path.join(td, "x.raw"))
        rng.standard_normal(D, dtype=np.float32).tofile(os.path.join(td, "emb.raw"))
        (rng.standard_normal(6144, dtype=np.float32) * 0.1).tofile(os.path.join(td, "lora.raw"))
        rng.standard_normal((1024, nctx), dtype=np.float32).tofile(os.path.join(td, "ctx.raw"))
        cmd = f"run {td}/x.raw {td}/emb.raw {td}/lora.raw {td}/ctx.raw {td}/out.raw {gh} {gw}\n"
        env = dict(os.environ, HXA_RUN_DBG="1")
        t0 = time.perf_counter()
        r = subprocess.run([exe, td, "0", str(NBLK)], input=cmd * (runs + 1) + "quit\n", capture_output=True, text=True,
                           timeout=900, env=env)
        wall = time.perf_counter() - t0
        done = [ln for ln in r.stdout.splitlines() if ln.startswith("done ")]
        if r.returncode != 0 or len(done) != runs + 1:
            raise RuntimeError(f"hxa_run failed ({r.returncode}): {r.stdout[-500:]} {r.stderr[-2000:]}")
        split = [ln for ln in r.stderr.splitlines() if ln.startswith("run: ")]
        blocks_ms = [float(ln.split("modulation+blocks ")[1].split(" ms")[0]) for ln in split][1:]
        out = np.fromfile(os.path.join(td, "out.raw"), np.float32)
        if out.size != D * gh * gw or not np.isfinite(out).all():
            raise RuntimeError("hxa_run output missing or non-finite")
    ms = float(np.median(blocks_ms))
    return {"modulation_plus_28_blocks_ms": round(ms, 2), "per_block_ms": round(ms / NBLK, 3),
            "run_ms_incl_file_io": [int(ln.split()[1]) for ln in done[1:]],
            "first_run_ms_incl_weight_conversion": int(done[0].split()[1]), "process_wall_s": round(wall, 1),
            "config": "hxa_run (megarun protocol), 28 fp16 blkNN.bin, 1536 tokens, 512 context tokens, mod on GPU"}


def _cpu_model():
    """The first CPU's model name with its family / model / stepping numbers and microcode from /proc/cpuinfo (a
    virtual machine may show a short model name; the numbers still identify the part), and the logical CPU count."""
    f = {}
    n = 0
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k = k.strip()
            if k == "processor":
                n += 1
            if k in ("model name", "cpu family", "model", "stepping", "microcode", "cpu MHz") and k not in f:
                f[k] = v.strip()
    except OSError:
        return "unknown"
    return (f"{f.get('model name', 'unknown')} (family {f.get('cpu family', '?')}, model {f.get('model', '?')}, "
            f"stepping {f.get('stepping', '?')}, microcode {f.get('microcode', '?')}, {f.get('cpu MHz', '?')} MHz; "
            f"{n} logical CPUs in the host)")


def cpu_baseline():
    """The oracle (C port of the reference block, built for this host with -march=native and OpenMP) on whole
    1536-token blocks, scaled to the 28-block step, and on one 1536 x 2048 x 8192 fp16 GEMM (double accumulation)."""
    from oracle import hxo
    flags = hxo.use_native()
    threads = hxo.set_threads(0)
    rng = np.random.default_rng(3)
    w = {}
    for k, (n, kk) in {"wq": (D, D), "wk": (D, D), "wv": (D, D), "wo": (D, D), "wcq": (D, D), "wck": (D, DC),
                       "wcv": (D, DC), "wco": (D, D), "w1": (F, D), "w2": (D, F)}.items():
        w[k] = (rng.standard_normal((n, kk), dtype=np.float32) * 0.02).astype(np.float16)
    w["gain"] = np.concatenate([np.full(128, 128 ** -0.5), np.ones(128), np.full(128, 128 ** -0.5), np.ones(128)]).astype(np.float32)
    x = rng.standard_normal((T, D), dtype=np.float32)
    ctx = rng.standard_normal((C_TXT, DC), dtype=np.float32).astype(np.float16)
    mod9 = (rng.standard_normal((9, D), dtype=np.float32) * 0.2)
    cos, sin = hxo.rope_anima(LAT[1] // 2, LAT[2] // 2)
    # bounded sample: whole 1536-token blocks (each feeding the next, as in a step) until ~12 s of CPU work
    nblk, t0 = 0, time.perf_counter()
    while nblk < NBLK and (nblk == 0 or time.perf_counter() - t0 < 12.0):
        x, _, _ = hxo.anima_block(x, ctx, mod9, cos, sin, w, H=H, F=F, gelu=1)
        nblk += 1
    tb = (time.perf_counter() - t0) / nblk
    A = rng.standard_normal((T, D), dtype=np.float32).astype(np.float16)
    hxo.gemm(A[:64], w["w1"])
    t0 = time.perf_counter()
    for _ in range(2):
        hxo.gemm(A, w["w1"])
    tg = (time.perf_counter() - t0) / 2
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = os.cpu_count()
    return {"value": round(1.0 / (NBLK * tb), 5), "unit": "steps/s", "cores": threads, "kind": "port",
            "sample": f"{nblk} chained 1536-token blocks on the C oracle ({tb:.2f} s each), scaled to the 28-block "
                      f"step; 2 GEMMs 1536x2048x8192",
            "block_ms": round(tb * 1e3, 1), "steps_per_s_batch4": round(1.0 / (4 * NBLK * tb), 6),
            "steps_per_s_batch4_basis": "4 x the batch-1 block time (the oracle block runs one image; the work is 4x)",
            "gemm_1536x2048x8192_gflops": round(2 * T * D * F / tg / 1e9, 1),
            "nproc": aff, "cpu_model": _cpu_model(), "threads": threads, "compiler": flags,
            "label": "baseline only"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="leave out the other DiT workloads, the kernel microbenchmarks and the ABI chain (for a "
                         "kernel trace of the step)")
    ap.add_argument("--workload", choices=sorted(EXTRA_DITS), default=None,
                    help="time only this other DiT workload and print its JSON (for a kernel trace of it)")
    ap.add_argument("--kernel-probe", type=int, default=0, metavar="REPS",
                    help="only launch one kernel family REPS times plus a copy calibration (for rocprofv3 --pmc)")
    ap.add_argument("--probe-family", default="gemm_splitk",
                    choices=["gemm_splitk", "gemm_pp_mlp_up", "gemm_pp_qkv_headnorm", "attention", "gemm_xattn_cross",
                             "linears_f16", "linears_q8", "linears_q4", "linear_split_f16", "linear_split_q8",
                             "linear_split_q4"])
    ap.add_argument("--abi-chain", action="store_true", help="only time the 28-block mega_block chain (hxa_run)")
    ap.add_argument("--clock-probe", action="store_true",
                    help="only measure the shader clock of the MLP-up GEMM (random / zero data, one workgroup) and of "
                         "the DiT step's kernels")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build targets a single MI355X (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    if a.kernel_probe:
        kernel_probe(a.kernel_probe, a.probe_family)
        return
    if a.clock_probe:
        clock_probe()
        return
    if a.abi_chain:
        print(json.dumps({"abi_chain": abi_chain()}), flush=True)
        return
    if a.workload:
        from hexanima_amd import hip
        hip.init(0)
        print(json.dumps({a.workload: EXTRA_DITS[a.workload]()}), flush=True)
        return
    info, ms_step = gpu_run(a.steps, a.warmup)
    from hexanima_amd import hip
    kernels, roof = kernel_breakdown(hip.lib(), hip)
    res = {
        "metric": "DiT denoise steps/s at 1536 tok (2B fp16, 2.9B q8); GEMM+attn % MFMA peak",
        "value": round(1000.0 / ms_step, 3),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) latent and text)",
        "config": {"workload": "2B-class fp16 DiT, 28 blocks, 1536 tokens, batch 1, 4-step Euler schedule",
                   "hidden": D, "heads": H, "mlp": F, "text_tokens": C_TXT, "latent": list(LAT), "global_batch": 1,
                   "seq_len": T, "parallelism": "single GPU"},
        "step_tflops": round(STEP_FLOPS / (ms_step * 1e-3) / 1e12, 1),
        "step_frac_of_fp16_peak": round(STEP_FLOPS / (ms_step * 1e-3) / PEAK_FP16, 4),
        "roofline": roof,
        "kernels": kernels,
        "device": info.get("name"),
    }
    print(json.dumps({"progress": "step, kernels done"}), file=sys.stderr, flush=True)
    if not a.no_extras:
        res.update(extra_dits())
        res["microbench"] = microbench()
        res["abi_chain"] = abi_chain()
        res["abi_chain"]["graph_step_ms_for_comparison"] = round(ms_step, 3)
    if not a.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
