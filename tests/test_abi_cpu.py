"""CPU-side checks of the C-ABI library: it loads, exports every function include/hexanima_hip.h declares, and its
host-only layout functions agree with the reference's byte layouts. No compute is launched here."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hexanima_hip.h")


MOSS_HEADER = os.path.join(ROOT, "include", "hexanima_moss.h")


def _declared(header=HEADER):
    src = open(header).read()
    return set(re.findall(r"^\s*(?:int|long|void\s*\*|const char\s*\*)\s*\**\s*(\w+)\s*\(", src, re.M))


@pytest.fixture(scope="module")
def hip():
    from hexanima_amd import hip as h
    h.lib()
    return h


def test_library_exports_every_declared_symbol(hip):
    out = subprocess.run(["nm", "-D", "--defined-only", hip.LIB_PATH], capture_output=True, text=True, check=True).stdout
    syms = {l.split()[-1] for l in out.splitlines() if l.strip()}
    decl = _declared()
    assert len(decl) >= 40
    assert decl <= syms, sorted(decl - syms)
    # the reference's three block-interface symbols (mega.idl:3-11, mega_imp.c:16-18, blk.c:186)
    assert {"mega_open", "mega_block", "mega_close"} <= syms
    # and the Python binding covers exactly the declared set
    assert set(hip.exported_symbols()) == decl


def test_moss_library_exports_the_reference_mega_block(hip):
    """libhexanima_moss.so exports mega_block (moss/hexagon/mega/blk.c:269, called mossrun.cpp:185) and nothing that
    would shadow libhexanima_hip.so's other entry points; it resolves mega_moss_block from libhexanima_hip.so."""
    path = os.path.join(os.path.dirname(hip.LIB_PATH), "libhexanima_moss.so")
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    syms = {l.split()[-1] for l in out.splitlines() if l.strip()} - {"_init", "_fini"}
    assert _declared(MOSS_HEADER) == {"mega_block"} and syms == {"mega_block"}, syms
    und = subprocess.run(["nm", "-D", "--undefined-only", path], capture_output=True, text=True, check=True).stdout
    assert "mega_moss_block" in und
    C.CDLL(path).mega_block  # loads, with libhexanima_hip.so found next to it


def test_pack_layout_matches_reference_matrix_bytes(hip):
    # an fp16 Anima pack holds the same ten matrices as blkNN.bin: 125829120 bytes before the gains (blk_wlayout.h:18)
    total, mats, voff = hip.pack_layout(0, 2048, 8192, 1024, 0, 0)
    assert voff == 125829120
    assert all(o % 256 == 0 for o, _ in mats) and voff % 256 == 0
    # q8: one int8 per weight + one fp16 scale per (32-row group, column) = 17/16 byte per weight (the reference
    # record stores each scale twice: 1152 B per 32x32 tile, export_all.py:10-18)
    t8, m8, v8 = hip.pack_layout(0, 2048, 8192, 1024, 1, 1)
    assert v8 == 125829120 // 2 * 17 // 16
    t4, m4, v4 = hip.pack_layout(1, 3072, 12288, 0, 1, 2)
    assert all(s >= 0 for _, s in m4)


@pytest.mark.parametrize("cb", [64, 32, 16])
def test_ktile_places_each_row_chunk_at_its_k_step(hip, cb):
    """The block-pack matrix order: the chunk of row n and k group g (64 B fp16, 32 B q8, 16 B q4) sits at
    (g * N + n) * chunk, so one 32-deep k step of all N rows is one contiguous slice; unktile inverts it."""
    N, K = 40, 96
    rm = np.random.default_rng(2).integers(0, 256, N * (K // 32) * cb, dtype=np.uint8)
    kt = hip.ktile(rm, N, K)
    for n in (0, 7, N - 1):
        for g in range(K // 32):
            assert np.array_equal(kt[(g * N + n) * cb:(g * N + n + 1) * cb], rm[(n * (K // 32) + g) * cb:][:cb])
    assert np.array_equal(hip.unktile(kt, N, K), rm)


def test_ws_bytes_and_init_without_gpu(hip):
    d = hip.BlockDims(0, 2048, 16, 8192, 256, 1024, 1536, 1, 1536, 0, 0, 1)
    # h, q|k, v^T, o, two split-K partials (fp16, 7 x [T][D] in total) + the MLP hidden [T][F] + cross k / v^T
    assert hip.lib().hxa_block_ws_bytes(C.byref(d)) >= 1536 * (14 * 2048 + 2 * 8192) + 4 * 256 * 2048
    if not os.path.exists("/dev/kfd"):
        rc = hip.lib().hxa_init(0)
        assert rc == -13 and "device" in hip.last_error()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    import importlib
    from hexanima_amd import hip as h
    monkeypatch.setattr(h, "LIB_PATH", str(tmp_path / "absent.so"))
    monkeypatch.setattr(h, "_lib", None)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        h.lib()


def test_host_programs_reject_bad_arguments_before_any_device_call(hip, tmp_path):
    """hxa_run (megarun protocol) and hxa_blk (blk_main harness) are built beside the library and fail cleanly on
    missing inputs; the GPU runs of both are in tests/test_gpu_runners.py."""
    d = os.path.dirname(hip.LIB_PATH)
    run, blk = os.path.join(d, "hxa_run"), os.path.join(d, "hxa_blk")
    r = subprocess.run([run], capture_output=True, text=True)
    assert r.returncode == 1 and "usage" in r.stderr
    r = subprocess.run([run, str(tmp_path), "0", "2"], capture_output=True, text=True)
    assert r.returncode == 1 and "cannot load" in r.stderr
    (tmp_path / "blk00.bin").write_bytes(b"\0" * 4096)
    r = subprocess.run([run, str(tmp_path), "0", "1"], capture_output=True, text=True)
    assert r.returncode == 1 and "not a block file" in r.stderr
    r = subprocess.run([blk, str(tmp_path)], capture_output=True, text=True)
    assert r.returncode == 1 and "missing" in r.stdout


def test_linear_split_choice_host_only(hip):
    """hxa_linear's K-slice choice is host logic (the tile model, no launch): the long-K N <= K shapes of the
    benchmark split (the forms measured fastest on MI355X), the wide and square ones run as one launch, and the
    workspace size follows the choice. Without a GPU the model takes 256 CUs, the MI355X count."""
    L = hip.lib()
    M = 1536
    want = {(2048, 8192, 0): 2, (2048, 8192, 1): 4, (2048, 8192, 2): 4, (2560, 10240, 1): 4, (2560, 10240, 2): 4,
            (6144, 2048, 1): 1, (2048, 2048, 1): 1, (8192, 2048, 1): 1, (7680, 2560, 0): 1}
    for (N, K, fmt), S in want.items():
        assert L.hxa_linear_split_k(M, N, K, fmt) == S, (N, K, fmt)
        assert L.hxa_linear_ws_bytes(M, N, K, fmt) == (S * M * N * 4 if S > 1 else 0)
        assert L.hxa_linear_split_k(M, N, K, fmt | hip.W_KTILED) == S
    assert L.hxa_linear_split_k(M, 2044, 8192, 1) == 1  # N % 8 != 0: no split form
    assert L.hxa_linear_split_k(0, 2048, 8192, 1) == 1
