"""Child process of test_zz_no_alloc.py::test_block_run_noalloc_first_call_captured (run in a fresh process, so that
the captured call is the process's first hxa_block_run_noalloc and the first launch of every kernel it uses).

hxa_init, then the first noalloc call is captured into a HIP graph (global capture mode: any call the runtime forbids
under capture invalidates it) and the graph is replayed three times, with eager work between the replays (an eager
noalloc call on other data, which leaves different contents in the shared static workspace, and an hxa_block_run).
Every replay must give the bits hxa_block_run gives with a caller workspace. Prints one line per step; exit code 0
on success."""
import ctypes as C
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def main() -> int:
    from hexanima_amd import hip
    from oracle import hxo
    from tests._helpers import f16
    from tests.test_gpu_block import cfg0_mod9, make_anima_pack

    hip.init(0)
    lib = hip.lib()
    rng = np.random.default_rng(606)
    D, F, T, fmt, C_, DC = 2048, 8192, 1536, 1, 256, 1024
    print(f"[child] int8 block D={D} T={T}: first noalloc call under graph capture", flush=True)
    img, _, H = make_anima_pack(hip, rng, D, F, DC, fmt)
    x = rng.standard_normal((T, D)).astype(np.float32)
    x2 = rng.standard_normal((T, D)).astype(np.float32)
    ctx = f16(rng.standard_normal((C_, DC)))
    mod = cfg0_mod9(D, rng)
    cos, sin = hxo.rope_anima(T // 32, 32)
    d = hip.BlockDims(0, D, H, F, C_, DC, T, 1, T, fmt, fmt, 1)
    pack, dctx, dmod, dcos, dsin = (hip.DeviceArray.from_numpy(a) for a in (img, ctx, mod, cos, sin))
    x0 = hip.DeviceArray.from_numpy(x)
    xw = hip.DeviceArray.from_numpy(x)   # the captured call's x (reset from x0 before every replay)
    xo = hip.DeviceArray.from_numpy(x2)  # other data for the eager calls between replays
    s = C.c_void_p()
    hip.check(lib.hxa_stream_create(C.byref(s)), "stream")
    hip.check(lib.hxa_stream_begin_capture(s, 0), "begin capture")
    rc = lib.hxa_block_run_noalloc(C.byref(d), pack.ptr, xw.ptr, dctx.ptr, dmod.ptr, dcos.ptr, dsin.ptr, 0, s)
    err = hip.last_error() if rc else ""
    ex = C.c_void_p()
    rc2 = lib.hxa_stream_end_capture(s, C.byref(ex))
    if rc != 0 or rc2 != 0:
        print(f"[child] capture failed: noalloc rc {rc} ({err}), end capture rc {rc2} ({hip.last_error()})", flush=True)
        return 1
    print("[child] captured", flush=True)
    # the reference: hxa_block_run with a caller workspace on the same input
    ws = hip.block_ws(d)
    xr = hip.DeviceArray.from_numpy(x)
    hip.check(lib.hxa_block_run(C.byref(d), pack.ptr, xr.ptr, dctx.ptr, dmod.ptr, dcos.ptr, dsin.ptr, ws.ptr, 0, None, 0,
                                None), "block_run")
    hip.sync()
    ref = xr.numpy()
    ok = True
    for rep in range(3):
        if rep == 1:  # eager noalloc call on other data: the static workspace now holds its buffers
            hip.check(lib.hxa_block_run_noalloc(C.byref(d), pack.ptr, xo.ptr, dctx.ptr, dmod.ptr, dcos.ptr, dsin.ptr, 0,
                                                None), "eager noalloc")
        if rep == 2:  # eager block run with a caller workspace
            hip.check(lib.hxa_block_run(C.byref(d), pack.ptr, xo.ptr, dctx.ptr, dmod.ptr, dcos.ptr, dsin.ptr, ws.ptr, 0,
                                        None, 0, None), "eager block_run")
        hip.sync()
        hip.check(lib.hxa_d2d(xw.ptr, x0.ptr, x.nbytes), "reset x")
        hip.check(lib.hxa_graph_launch(ex, s), "graph launch")
        hip.check(lib.hxa_stream_sync(s), "sync")
        got = xw.numpy()
        same = bool(np.array_equal(got.view(np.uint32), ref.view(np.uint32)))
        changed = not np.array_equal(got, x)
        print(f"[child] replay {rep}: bit-identical to hxa_block_run {same}, x changed {changed}", flush=True)
        ok = ok and same and changed and bool(np.isfinite(got).all())
    hip.check(lib.hxa_graph_exec_destroy(ex), "graph destroy")
    hip.check(lib.hxa_stream_destroy(s), "stream destroy")
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())
