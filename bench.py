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


def gpu_run(steps, warmup):
    from hexanima_amd import hip
    hip.init(0)
    L = hip.lib()
    info = hip.device_info()
    bd = hip.BlockDims(0, D, H, F, C_TXT, DC, 0, 1, 0, hip.W_F16, hip.W_F16, 1)
    cfg = hip.DitCfg(bd, NBLK, LAT[0], LAT[1], LAT[2], 256, 0)
    dit = C.c_void_p()
    hip.check(L.hxa_dit_create(C.byref(cfg), 2024, C.byref(dit)), "dit_create")
    rng = np.random.default_rng(1)
    lat = rng.standard_normal((1,) + LAT).astype(np.float32)
    ctx = rng.standard_normal((1, C_TXT, DC)).astype(np.float32)
    hip.check(L.hxa_dit_set_inputs(dit, lat.ctypes.data, ctx.ctypes.data), "set_inputs")
    st = L.hxa_dit_stream(dit)
    sig = [1.0, 0.75, 0.5, 0.25, 0.0]

    def ev():
        p = C.c_void_p()
        hip.check(L.hxa_event_create(C.byref(p)), "event")
        return p

    e0, e1 = ev(), ev()
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
    ms_step = max(ms.value, wall * 1e3) / steps
    out = np.zeros_like(lat)
    hip.check(L.hxa_dit_get_latent(dit, out.ctypes.data), "latent")
    if not np.isfinite(out).all():
        raise RuntimeError("non-finite latent")
    L.hxa_dit_destroy(dit)

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
    for _ in range(5):
        up()
    reps = 50
    hip.check(L.hxa_event_record(e0, s), "rec")
    for _ in range(reps):
        up()
    hip.check(L.hxa_event_record(e1, s), "rec")
    hip.check(L.hxa_event_elapsed_ms(e0, e1, C.byref(ms)), "elapsed")
    up_ms = ms.value / reps
    L.hxa_stream_destroy(s)
    return info, ms_step, up_ms


def q8_dit_run(steps=10, warmup=2):
    """The 2.9B-class q8 DiT step (28 blocks, hidden 2560, 20 heads, MLP 10240, every block linear int8 with fp16
    group-32 scales; norms and modulation fp16), same latent / text shapes: ms per graph-replayed Euler step."""
    from hexanima_amd import hip
    L = hip.lib()
    Dq, Hq, Fq = 2560, 20, 10240
    bd = hip.BlockDims(0, Dq, Hq, Fq, C_TXT, DC, 0, 1, 0, hip.W_Q8, hip.W_Q8, 1)
    cfg = hip.DitCfg(bd, NBLK, LAT[0], LAT[1], LAT[2], 256, 0)
    dit = C.c_void_p()
    hip.check(L.hxa_dit_create(C.byref(cfg), 2025, C.byref(dit)), "dit_create q8")
    rng = np.random.default_rng(2)
    lat = rng.standard_normal((1,) + LAT).astype(np.float32)
    ctx = rng.standard_normal((1, C_TXT, DC)).astype(np.float32)
    hip.check(L.hxa_dit_set_inputs(dit, lat.ctypes.data, ctx.ctypes.data), "set_inputs q8")
    st = L.hxa_dit_stream(dit)
    sig = [1.0, 0.75, 0.5, 0.25, 0.0]
    e0, e1 = C.c_void_p(), C.c_void_p()
    hip.check(L.hxa_event_create(C.byref(e0)), "event")
    hip.check(L.hxa_event_create(C.byref(e1)), "event")
    for i in range(warmup):
        hip.check(L.hxa_dit_step(dit, sig[i % 4], sig[i % 4 + 1], 1), "step q8")
    hip.check(L.hxa_event_record(e0, st), "rec")
    for i in range(steps):
        hip.check(L.hxa_dit_step(dit, sig[i % 4], sig[i % 4 + 1], 1), "step q8")
    hip.check(L.hxa_event_record(e1, st), "rec")
    hip.check(L.hxa_stream_sync(st), "sync")
    ms = C.c_float()
    hip.check(L.hxa_event_elapsed_ms(e0, e1, C.byref(ms)), "elapsed")
    out = np.zeros_like(lat)
    hip.check(L.hxa_dit_get_latent(dit, out.ctypes.data), "latent q8")
    L.hxa_dit_destroy(dit)
    if not np.isfinite(out).all():
        raise RuntimeError("non-finite q8 latent")
    blk = 2 * T * Dq * (3 * Dq) + 3 * 2 * T * Dq * Dq + 2 * C_TXT * DC * 2 * Dq + 2 * 2 * T * Dq * Fq \
        + 4 * T * T * Dq + 4 * T * C_TXT * Dq
    ms_step = ms.value / steps
    return {"steps_per_s": round(1000.0 / ms_step, 3), "ms_per_step": round(ms_step, 4),
            "step_tflops": round(NBLK * blk / (ms_step * 1e-3) / 1e12, 1),
            "config": "28 blocks, hidden 2560, 20 heads, MLP 10240, int8 g32 block linears, 1536 image + 256 text tokens"}


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
    ap.add_argument("--kernel-probe", type=int, default=0, metavar="REPS",
                    help="only launch the dominant kernel REPS times plus a copy calibration (for rocprofv3 --pmc)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build targets a single MI355X (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    if a.kernel_probe:
        kernel_probe(a.kernel_probe)
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
        "roofline": {"kernel": "gemm_kernel (fp16 k-tiled W, GELU epilogue) MLP up 1536x2048x8192", "bound": "mfma",
                     "achieved": round(up_tf / 1e12, 1), "peak": PEAK_FP16 / 1e12, "unit": "TFLOP/s",
                     "frac": round(up_tf / PEAK_FP16, 4), "traffic": traffic, "avg_launch_us": round(up_ms * 1e3, 2)},
        "device": info.get("name"),
    }
    res["q8_2p9b_dit"] = q8_dit_run()
    if not a.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
