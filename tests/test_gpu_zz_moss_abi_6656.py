"""The MOSS-class block through the reference's own symbol at its full shape: two chained blocks through
libhexanima_moss.so's mega_block (mossrun.cpp:182-188, MODE 0; FIRST on the first, REL on the second) at 6656 tokens,
6144 image (a 64 x 96 patch grid) + 512 text, on synthetic export_moss.py packs (q8 records with the rapid-moss LoRA,
hidden 3072, MLP 8192), against the oracle with the LoRA term. The modulation is N(0, 0.2), so the gates are O(0.1 -
1) and the blocks' updates are a large part of x (printed). Tolerance about 3x the error measured on MI355X. The
oracle takes about a minute on 16 host threads; collected after the other GPU tests."""
import ctypes as C
import os
import time

import numpy as np
import pytest

from oracle import hxo
from tests._helpers import rel
from tests.test_gpu_block import MOSS_META, _moss_blk_file, _mossrun_layout, metrics_line

pytestmark = pytest.mark.gpu


def test_mega_block_moss_abi_6656tok_two_blocks():
    from hexanima_amd import hip

    hip.init(0)
    lib = hip.lib()
    hxo.set_threads(0)
    print("[case] MOSS mega_block ABI with LoRA, 2 chained blocks, T=6656 (6144 + 512)", flush=True)
    moss = C.CDLL(os.path.join(os.path.dirname(hip.LIB_PATH), "libhexanima_moss.so"))
    moss.mega_block.restype = C.c_int
    moss.mega_block.argtypes = [C.c_uint64, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_void_p,
                                C.c_int, C.c_void_p]
    rng = np.random.default_rng(66)
    D, F, gh, gw, ntxt = 3072, 8192, 64, 96, 512
    NV = gh * gw + ntxt
    T = (NV + 31) // 32 * 32
    files = [_moss_blk_file(rng) for _ in range(2)]
    offs, total = _mossrun_layout(T)
    blob = np.zeros(total, np.uint8)
    x = np.zeros((T, D), np.float32)
    x[:NV] = rng.standard_normal((NV, D))
    bands = (1.0 / 10000.0 ** (np.arange(16) / 16)).astype(np.float32)
    cs, sn = hxo.rope_moss(gh, gw, ntxt, bands)
    cos, sin = np.zeros((T, 64), np.float32), np.zeros((T, 64), np.float32)
    cos[:NV], sin[:NV] = cs, sn
    blob[offs["X"]:offs["X"] + T * D * 4] = hxo.x32_tile(x).view(np.uint8)
    for nm, tab in (("COS", cos), ("SIN", sin)):
        t = np.ascontiguousarray(tab.reshape(T // 32, 32, 2, 32).transpose(0, 2, 1, 3)).astype(np.float32)
        blob[offs[nm]:offs[nm] + t.nbytes] = t.view(np.uint8).reshape(-1)
    mods = [(rng.standard_normal((6, D)) * 0.2).astype(np.float32) for _ in range(2)]
    meta = np.zeros(len(MOSS_META), np.int32)
    for k, v in offs.items():
        meta[MOSS_META.index(k)] = v
    for k, v in (("NTOK", T), ("NVALID", NV), ("NW", 3), ("MODE", 0), ("NCB", 96), ("WOFF", 0)):
        meta[MOSS_META.index(k)] = v
    h = C.c_uint64()
    hip.check(lib.mega_open(b"", C.byref(h)), "mega_open")
    try:
        hip.check(lib.hxa_register(h, 100, blob.ctypes.data, blob.nbytes, hip.KIND_BLOB), "register blob")
        for i, (wf, _) in enumerate(files):
            hip.check(lib.hxa_register(h, 300 + i, wf.ctypes.data, wf.nbytes, hip.KIND_WEIGHTS_MOSS), "register w")
        rc = C.c_int(0)
        times = np.full(32, -1, np.int32)
        for i in range(2):
            meta[MOSS_META.index("FIRST")], meta[MOSS_META.index("REL")] = int(i == 0), int(i == 1)
            t0 = time.time()
            r = moss.mega_block(h.value, meta.ctypes.data, len(MOSS_META), 300 + i, 100, mods[i].ctypes.data,
                                mods[i].nbytes, times.ctypes.data, 32, C.byref(rc))
            assert r == 0 and rc.value == 0, hip.last_error()
            print(f"block {i}: times (us) {times[:8].tolist()}, call {1e3 * (time.time() - t0):.0f} ms", flush=True)
        got = hxo.x32_untile(blob[offs["X"]:offs["X"] + T * D * 4].view(np.float32).copy(), T, D)
        t0 = time.time()
        ref = x
        for (_, w), m in zip(files, mods):
            ref, _, _ = hxo.moss_block(ref, m, cos, sin, w, H=24, F=F, nvalid=NV)
        print(f"oracle 2 blocks in {time.time() - t0:.1f} s", flush=True)
        share = rel(ref[:NV] - x[:NV], x[:NV])
        r_, c, mx = metrics_line(got[:NV], ref[:NV], x[:NV])
        print(f"MOSS ABI 6656 tokens: rel err on delta {r_:.2e} cos {c:.8f} max abs {mx:.2e}; the blocks change x "
              f"by {share:.3f} (relative)", flush=True)
        assert np.isfinite(got).all()
        assert share > 0.2  # measured 1.43
        assert r_ < 2.2e-3 and c > 1 - 2.2e-3 ** 2 and mx < 3.2e-2  # measured 7.4e-4, 1.0e-2
    finally:
        lib.mega_close(h)
