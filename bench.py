"""Benchmark: DiT denoise steps/s of the 2B-class fp16 DiT at 1536 tokens on one MI355X.

Workload: 28 Anima-structure blocks (hidden 2048, 16 heads x 128, MLP 8192, tanh GELU, 256 text tokens of width
1024), patch embed 64 -> 2048, final adaLN + linear 2048 -> 64, batch 1, latent 16 x 96 x 64 (1536 tokens),
random N(0, 0.02) weights, N(0, 1) latent and text. One step = one flow-matching Euler step (timestep embedding,
28 x modulation, patch embed, 28 blocks, final layer, update), replayed from a captured HIP graph with the sigma
schedule 1.0, 0.75, 0.5, 0.25 -> 0 cycled.

Prints one JSON line. `roofline` is for the dominant kernel (the MLP up-projection GEMM with GELU epilogue,
1536 x 2048 x 8192, the largest launch of the step), timed with HIP events on the stream it is launched on.
`cpu_baseline` times the CPU oracle (a port of the reference block) on one block and scales to a step.
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
BLOCK_FLOPS = 2 * T * D * (3 * D) + 2 * T * D * D + 2 * T * D * D + 2 * C_TXT * DC * (2 * D) + 2 * T * D * D \
    + 2 * T * D * F * 2 + 4 * T * T * D + 4 * T * C_TXT * D
STEP_FLOPS = NBLK * BLOCK_FLOPS + 2 * T * 64 * D + 2 * T * D * 64
UP_FLOPS = 2 * T * D * F


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
    L = hip.lib()
    info = hip.device_info()
    bd = hip.BlockDims(0, D, H, F, C_TXT, DC, 0, 1, 0, hip.W_F16, hip.W_F16, 1)
    ms_step = dit_ms(bd, NBLK, (1,) + LAT, (1, C_TXT, DC), 0, steps, warmup, 2024, wall_check=True)

    # dominant kernel: MLP up-projection GEMM with the GELU epilogue (one launch per block per step)
    s = C.c_void_p()
    hip.check(L.hxa_stream_create(C.byref(s)), "stream")
    A = hip.DeviceArray((T, D), np.float16)
    W = hip.DeviceArray((F, D), np.float16)
    O = hip.DeviceArray((T, F), np.float16)
    hip.check(L.hxa_fill_normal(A.ptr, 1, T * D, 11, 0.0, 1.0, s), "fill")
    hip.check(L.hxa_fill_normal(W.ptr, 1, F * D, 12, 0.0, 0.02, s), "fill")

    def up():
        hip.check(L.hxa_gemm(A.ptr, D, T, WFMT, W.ptr, None, None, F, D, 1, hip.EPI_GELU_TANH, O.ptr, F, 0, None, 0,
                             None, None, 0, 0, s), "gemm")
    up_ms = _time_launches(L, hip, up, s, reps=50)
    L.hxa_stream_destroy(s)
    pk = hip.gemm_pick(T, F, D, WFMT, 1, hip.EPI_GELU_TANH)
    info["up_kernel"] = (f"{'gemm_pp_kernel' if pk['waves'] == 9 else 'gemm_kernel'} {pk['bm']}x{pk['bn']}"
                         f" ({8 if pk['waves'] == 9 else pk['waves']} waves)")
    return info, ms_step, up_ms


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
      [-127, 127] / int4 uniform in [-8, 7], group-32 fp16 scales 0.02/127, pack layout), beside fp16 weights;
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
    hip.check(L.hxa_fill_const(Sb.ptr, 1, 320 * 10240, 0.02 / 127, s), "fill")
    # the 2B block's projections in each format, and the 2.9B-class block's (hidden 2560, MLP 10240) in fp16 / int8
    for key, shapes, fmts in (("linear_m1536", ((2048, 6144), (2048, 2048), (2048, 8192), (8192, 2048)),
                               (("fp16", hip.W_F16), ("q8", hip.W_Q8), ("q4", hip.W_Q4))),
                              ("linear_m1536_2p9b", ((2560, 7680), (2560, 2560), (2560, 10240), (10240, 2560)),
                               (("fp16", hip.W_F16), ("q8", hip.W_Q8)))):
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
                row[f"{K}x{N}"] = _rate(2.0 * M * N * K, _time_launches(L, hip, run, s))
            res[key][name] = row
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

    def blk():
        hip.check(L.hxa_block_run(C.byref(bd), pack.ptr, x.ptr, ctx.ptr, mod.ptr, cos.ptr, sin.ptr, ws.ptr, 0, None, 0,
                                  s), "block")
    res["block_2b_fp16_1536tok"] = _rate(BLOCK_FLOPS, _time_launches(L, hip, blk, s, reps=10, warm=2))
    hip.check(L.hxa_stream_sync(s), "sync")
    L.hxa_stream_destroy(s)
    return res


def kernel_probe(reps):
    """Launches only the dominant kernel (MLP-up GEMM, `reps` times) and a 256 MiB device-to-device copy (3 times,
    the byte-count calibration of the FETCH_SIZE / WRITE_SIZE counters), for `rocprofv3 --pmc` passes."""
    from hexanima_amd import hip
    hip.init(0)
    L = hip.lib()
    s = C.c_void_p()
    hip.check(L.hxa_stream_create(C.byref(s)), "stream")
    A = hip.DeviceArray((T, D), np.float16)
    W = hip.DeviceArray((F, D), np.float16)
    O = hip.DeviceArray((T, F), np.float16)
    hip.check(L.hxa_fill_normal(A.ptr, 1, T * D, 11, 0.0, 1.0, s), "fill")
    hip.check(L.hxa_fill_normal(W.ptr, 1, F * D, 12, 0.0, 0.02, s), "fill")
    for _ in range(reps):
        hip.check(L.hxa_gemm(A.ptr, D, T, WFMT, W.ptr, None, None, F, D, 1, hip.EPI_GELU_TANH, O.ptr, F, 0, None, 0,
                             None, None, 0, 0, s), "gemm")
    nb = 256 << 20
    src = hip.DeviceArray((nb,), np.uint8)
    dst = hip.DeviceArray((nb,), np.uint8)
    hip.check(L.hxa_stream_sync(s), "sync")
    hip.check(L.hxa_memset(src.ptr, 1, nb), "memset")
    for _ in range(3):
        hip.check(L.hxa_d2d(dst.ptr, src.ptr, nb), "copy")
    hip.check(L.hxa_stream_sync(s), "sync")
    print(f"kernel probe: {reps} x gemm {T}x{D}x{F} GELU, 3 x copy {nb} B", flush=True)


def cpu_baseline():
    """The oracle (C port of the reference block, OpenMP) on one 1536-token block, scaled to a 28-block step."""
    from oracle import hxo
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
    # bounded sample: whole 1536-token blocks (each feeding the next, as in a step) until ~10 s of CPU work
    nblk, t0 = 0, time.perf_counter()
    while nblk < NBLK and (nblk == 0 or time.perf_counter() - t0 < 10.0):
        x, _, _ = hxo.anima_block(x, ctx, mod9, cos, sin, w, H=H, F=F, gelu=1)
        nblk += 1
    tb = (time.perf_counter() - t0) / nblk
    return {"value": round(1.0 / (NBLK * tb), 5), "unit": "steps/s", "cores": threads, "kind": "port",
            "sample": f"{nblk} chained 1536-token blocks on the C oracle ({tb:.2f} s each), scaled to the 28-block step"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="leave out the other DiT workloads and the kernel microbenchmarks (for a kernel trace of the step)")
    ap.add_argument("--workload", choices=sorted(EXTRA_DITS), default=None,
                    help="time only this other DiT workload and print its JSON (for a kernel trace of it)")
    ap.add_argument("--kernel-probe", type=int, default=0, metavar="REPS",
                    help="only launch the dominant kernel REPS times plus a copy calibration (for rocprofv3 --pmc)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build targets a single MI355X (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    if a.kernel_probe:
        kernel_probe(a.kernel_probe)
        return
    if a.workload:
        from hexanima_amd import hip
        hip.init(0)
        print(json.dumps({a.workload: EXTRA_DITS[a.workload]()}), flush=True)
        return
    info, ms_step, up_ms = gpu_run(a.steps, a.warmup)
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic_gemm_mlp_up_1536x2048x8192.txt")
    if os.path.exists(tpath):  # rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated (see that file)
        for line in open(tpath):
            if line.startswith("hbm_bytes_per_launch:"):
                traffic = int(line.split(":")[1])
    up_tf = UP_FLOPS / (up_ms * 1e-3)
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
        "roofline": {"kernel": f"{info['up_kernel']}, fp16 k-tiled W, GELU epilogue: MLP up {T}x{D}x{F}", "bound": "mfma",
                     "achieved": round(up_tf / 1e12, 1), "peak": PEAK_FP16 / 1e12, "unit": "TFLOP/s",
                     "frac": round(up_tf / PEAK_FP16, 4), "traffic": traffic, "avg_launch_us": round(up_ms * 1e3, 2)},
        "device": info.get("name"),
    }
    if not a.no_extras:
        res.update(extra_dits())
        res["microbench"] = microbench()
    if not a.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
