"""hxa_block_run_noalloc (no counterpart in the reference; for callers that cannot allocate device memory): the block
run through the library's static device workspace gives the same bits as hxa_block_run with a caller workspace,
on two calls in a row, the second with a smaller input (so the second runs on a workspace holding the first call's
data), and a block whose workspace exceeds the static maximum is an argument error that launches nothing."""
import ctypes as C

import numpy as np
import pytest

from oracle import hxo
from tests._helpers import f16
from tests.test_gpu_block import cfg0_mod9, make_anima_pack

pytestmark = pytest.mark.gpu


def _hip():
    from hexanima_amd import hip
    hip.init()
    return hip


def _inputs(hip, rng, D, F, T, fmt, C_=256, DC=1024):
    img, _, H = make_anima_pack(hip, rng, D, F, DC, fmt)
    x = rng.standard_normal((T, D)).astype(np.float32)
    ctx = f16(rng.standard_normal((C_, DC)))
    mod = cfg0_mod9(D, rng)
    gh = T // 32
    cos, sin = hxo.rope_anima(gh, 32)
    d = hip.BlockDims(0, D, H, F, C_, DC, T, 1, T, fmt, fmt, 1)
    dev = [hip.DeviceArray.from_numpy(a) for a in (img, ctx, mod, cos, sin)]
    return d, x, dev


def _run(hip, d, x, dev, noalloc):
    dx = hip.DeviceArray.from_numpy(x)
    pack, ctx, mod, cos, sin = (a.ptr for a in dev)
    lib = hip.lib()
    if noalloc:
        rc = lib.hxa_block_run_noalloc(C.byref(d), pack, dx.ptr, ctx, mod, cos, sin, 0, None)
    else:
        ws = hip.block_ws(d)
        rc = lib.hxa_block_run(C.byref(d), pack, dx.ptr, ctx, mod, cos, sin, ws.ptr, 0, None, 0, None)
    hip.check(rc, "noalloc block" if noalloc else "block")
    hip.sync()
    return dx.numpy()


def test_block_run_noalloc_matches_block_run():
    hip = _hip()
    lib = hip.lib()
    rng = np.random.default_rng(404)
    # first call: the 2B-class int8 block at 1536 tokens (108 MiB of workspace, the dequantisation slots included);
    # second call: an fp16 block at 512 tokens, on a workspace still holding the first call's buffers
    for D, F, T, fmt in ((2048, 8192, 1536, 1), (2048, 8192, 512, 0)):
        print(f"[case] noalloc block D={D} F={F} T={T} fmt={fmt}", flush=True)
        d, x, dev = _inputs(hip, rng, D, F, T, fmt)
        assert lib.hxa_block_ws_bytes(C.byref(d)) <= 160 << 20
        got = _run(hip, d, x, dev, noalloc=True)
        ref = _run(hip, d, x, dev, noalloc=False)
        assert np.isfinite(got).all() and not np.array_equal(got, x)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # a workspace beyond the static maximum (4 images of 1536 tokens: 272 MiB) is refused before any launch
    d4 = hip.BlockDims(0, 2048, 16, 8192, 256, 1024, 1536, 4, 1536, 0, 0, 1)
    assert lib.hxa_block_ws_bytes(C.byref(d4)) > 160 << 20
    dummy = hip.DeviceArray((256,), np.uint8, zero=True)
    rc = lib.hxa_block_run_noalloc(C.byref(d4), dummy.ptr, dummy.ptr, dummy.ptr, dummy.ptr, dummy.ptr, dummy.ptr, 0, None)
    assert rc == -12 and "static scratch" in hip.last_error()


def test_block_run_noalloc_first_call_captured():
    """The process's first noalloc call made under HIP graph capture (global mode), then replayed three times with
    eager work between the replays, gives hxa_block_run's bits each time. Runs in a child process, so the captured
    call is the first of its process whatever ran before this test (tests/_noalloc_capture.py)."""
    import os
    import subprocess
    import sys
    print("[case] noalloc first call under graph capture (child process)", flush=True)
    child = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_noalloc_capture.py")
    r = subprocess.run([sys.executable, "-u", child], capture_output=True, text=True, timeout=110)
    print(r.stdout[-3000:], r.stderr[-3000:], flush=True)
    assert r.returncode == 0
    assert r.stdout.count("bit-identical to hxa_block_run True") == 3
