"""ctypes binding of libhexanima_hip.so (include/hexanima_hip.h) plus small device-memory helpers.

There is no CPU fallback: every call goes to the HIP library, and importing a function that needs it raises
``RuntimeError`` when the library has not been built.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhexanima_hip.so")

P, I, L, F = C.c_void_p, C.c_int, C.c_long, C.c_float
SZ, U64 = C.c_size_t, C.c_uint64

# constants of the C-ABI
W_F16, W_Q8, W_Q4 = 0, 1, 2
W_KTILED = 16  # OR'ed into a format: matrix stored k-tiled, [K/32][N][chunk]
EPI_STORE, EPI_GELU_TANH, EPI_GELU_ERF, EPI_RESADD, EPI_STORE_T, EPI_SITU, EPI_PARTIAL, EPI_RESADD_SPLIT2, EPI_PARTIAL_F32 = range(9)
KIND_WEIGHTS_ANIMA, KIND_BLOB, KIND_WEIGHTS_MOSS = 0, 1, 2
E_NAMES = {0: "OK", -1: "RESOURCE", -2: "LOCK", -5: "WEIGHTS", -6: "NOBLOB", -7: "BLOB", -10: "META", -11: "MODE",
           -12: "ARG", -13: "HIP"}


class HxaError(RuntimeError):
    def __init__(self, rc: int, msg: str):
        super().__init__(f"hexanima_hip error {rc} ({E_NAMES.get(rc, '?')}): {msg}")
        self.rc = rc


class BlockDims(C.Structure):
    _fields_ = [("kind", I), ("D", I), ("H", I), ("F", I), ("C", I), ("DC", I), ("T", I), ("batch", I), ("nvalid", I),
                ("fmt_attn", I), ("fmt_mlp", I), ("gelu", I), ("round_ref", I)]


class DitCfg(C.Structure):
    _fields_ = [("blk", BlockDims), ("nblocks", I), ("lat_c", I), ("lat_h", I), ("lat_w", I), ("temb", I),
                ("ntxt_in", I), ("form", I)]


_SIGS = {
    "mega_open": (I, [C.c_char_p, C.POINTER(U64)]),
    "mega_close": (I, [U64]),
    "mega_block": (I, [U64, P, I, I, I, P, I, P, I, P]),
    "mega_moss_block": (I, [U64, P, I, I, I, P, I, P, I, P]),
    "hxa_register": (I, [U64, I, P, SZ, I]),
    "hxa_unregister": (I, [U64, I]),
    "hxa_anima_modulation": (I, [U64, P, I, P, P, P]),
    "hxa_last_error": (C.c_char_p, []),
    "hxa_version": (C.c_char_p, []),
    "hxa_init": (I, [I]),
    "hxa_malloc": (I, [C.POINTER(P), SZ]),
    "hxa_free": (I, [P]),
    "hxa_h2d": (I, [P, P, SZ]),
    "hxa_d2h": (I, [P, P, SZ]),
    "hxa_d2d": (I, [P, P, SZ]),
    "hxa_memset": (I, [P, I, SZ]),
    "hxa_sync": (I, []),
    "hxa_stream_create": (I, [C.POINTER(P)]),
    "hxa_stream_destroy": (I, [P]),
    "hxa_stream_sync": (I, [P]),
    "hxa_event_create": (I, [C.POINTER(P)]),
    "hxa_event_destroy": (I, [P]),
    "hxa_event_record": (I, [P, P]),
    "hxa_stream_wait_event": (I, [P, P]),
    "hxa_event_elapsed_ms": (I, [P, P, C.POINTER(F)]),
    "hxa_stream_begin_capture": (I, [P, I]),
    "hxa_stream_end_capture": (I, [P, C.POINTER(P)]),
    "hxa_graph_launch": (I, [P, P]),
    "hxa_graph_exec_destroy": (I, [P]),
    "hxa_device_info": (I, [C.POINTER(I), C.POINTER(I), C.POINTER(SZ), C.c_char_p, I]),
    "hxa_clock_record": (I, [I, P, L]),
    "hxa_gemm": (I, [P, L, I, I, P, P, P, I, I, I, I, P, L, L, P, L, P, P, L, I, P]),
    "hxa_resadd_norm_mod": (I, [P, L, I, I, P, L, P, P, P, P, F, P, L, P]),
    "hxa_gemm_headnorm": (I, [P, L, I, I, P, P, P, I, I, P, L, P, L, I, I, P, P, I, P, P, I, P]),
    "hxa_gemm_tile": (I, [P, L, I, I, P, P, P, I, I, I, I, P, L, L, P, L, P, I, I, I, P]),
    "hxa_gemm_pick": (I, [I, I, I, I, I, I, I, P, P, P, P]),
    "hxa_linear": (I, [P, L, I, I, P, P, P, I, I, P, L, P, L, P]),
    "hxa_linear_split_k": (I, [I, I, I, I]),
    "hxa_linear_ws_bytes": (L, [I, I, I, I]),
    "hxa_sum_partials": (I, [P, I, L, L, I, I, P, L, P]),
    "hxa_attention": (I, [P, L, P, L, P, L, P, L, I, I, I, I, I, L, L, L, L, P]),
    "hxa_norm_mod": (I, [P, L, I, I, P, P, P, F, P, L, P]),
    "hxa_cross_attention_fused": (I, [P, L, I, I, I, P, I, I, P, P, L, P, L, I, I, L, L, P, L, P]),
    "hxa_rmsrope": (I, [P, P, P, P, L, I, I, P, P, I, P]),
    "hxa_resadd2": (I, [P, L, P, P, L, I, I, P, P]),
    "hxa_dequant": (I, [I, P, P, P, I, I, P, P]),
    "hxa_fill_normal": (I, [P, I, SZ, U64, F, F, P]),
    "hxa_fill_uniform_int": (I, [P, I, SZ, U64, I, I, P]),
    "hxa_fill_const": (I, [P, I, SZ, F, P]),
    "hxa_quantize": (I, [P, I, I, I, P, P, P]),
    "hxa_x32_to_rows": (I, [P, P, I, I, P]),
    "hxa_rows_to_x32": (I, [P, P, I, I, P]),
    "hxa_pack_layout": (L, [I, I, I, I, I, I, C.POINTER(L), I]),
    "hxa_block_ws_bytes": (L, [C.POINTER(BlockDims)]),
    "hxa_block_run": (I, [C.POINTER(BlockDims), P, P, P, P, P, P, P, I, C.POINTER(I), I, P]),
    "hxa_block_ws_buf": (P, [C.POINTER(BlockDims), P, I, C.POINTER(L)]),
    "hxa_block_run_noalloc": (I, [C.POINTER(BlockDims), P, P, P, P, P, P, I, P]),
    "hxa_dit_create": (I, [C.POINTER(DitCfg), U64, C.POINTER(P)]),
    "hxa_dit_destroy": (I, [P]),
    "hxa_dit_set_inputs": (I, [P, P, P]),
    "hxa_dit_get_latent": (I, [P, P]),
    "hxa_dit_step": (I, [P, F, F, I]),
    "hxa_dit_velocity": (I, [P, F, P]),
    "hxa_dit_moss_step": (I, [P, F, I]),
    "hxa_dit_step_lowres": (I, [P, F, F, I, I]),
    "hxa_dit_moss_step_lowres": (I, [P, F, F, I]),
    "hxa_dit_export": (L, [P, I, P, SZ]),
    "hxa_dit_import": (I, [P, I, P, SZ]),
    "hxa_dit_load_block": (I, [P, I, P, SZ]),
    "hxa_dit_load_moss_block": (I, [P, I, P, SZ]),
    "hxa_dit_load_anima_glue": (I, [P, P, SZ]),
    "hxa_dit_load_moss_glue": (I, [P, P, SZ]),
    "hxa_dit_stream": (P, [P]),
}
_lib = None


def lib():
    """Load the HIP library (raises when it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m hexanima_amd.build` "
                               "(there is no CPU fallback)")
        lb = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(lb, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lb
    return _lib


def exported_symbols():
    return list(_SIGS)


def last_error() -> str:
    return (lib().hxa_last_error() or b"").decode()


def check(rc: int, what: str = ""):
    if rc != 0:
        raise HxaError(rc, f"{what}: {last_error()}")


_inited = False


def init(device: int = 0):
    global _inited
    if not _inited:
        check(lib().hxa_init(device), "hxa_init")
        _inited = True


def device_info():
    init()
    cu, clk, mem = I(), I(), SZ()
    name = C.create_string_buffer(256)
    check(lib().hxa_device_info(C.byref(cu), C.byref(clk), C.byref(mem), name, 256), "device_info")
    return {"num_cu": cu.value, "clock_khz": clk.value, "mem_bytes": mem.value, "name": name.value.decode()}


def gemm_pick(M, N, K, fmt, ksplit=1, epi=0, norm_cols=0):
    """the tile hxa_gemm chooses: {'bm', 'bn', 'waves' (9 = ping-pong kernel), 'rounds'}"""
    init()
    bm, bn, w, r = I(), I(), I(), I()
    check(lib().hxa_gemm_pick(M, N, K, fmt, ksplit, epi, norm_cols, C.byref(bm), C.byref(bn), C.byref(w), C.byref(r)),
          "gemm_pick")
    return {"bm": bm.value, "bn": bn.value, "waves": w.value, "rounds": r.value}


class DeviceArray:
    """A device allocation with a numpy-like shape / dtype; freed when garbage collected."""

    def __init__(self, shape, dtype, zero: bool = False):
        init()
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = P()
        check(lib().hxa_malloc(C.byref(p), max(self.nbytes, 1)), "hxa_malloc")
        self.ptr = p.value
        if zero:
            check(lib().hxa_memset(self.ptr, 0, max(self.nbytes, 1)), "hxa_memset")

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        if a.nbytes:
            check(lib().hxa_h2d(d.ptr, a.ctypes.data, a.nbytes), "hxa_h2d")
        return d

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.nbytes, self.nbytes)
        check(lib().hxa_h2d(self.ptr, a.ctypes.data, a.nbytes), "hxa_h2d")

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            check(lib().hxa_d2h(out.ctypes.data, self.ptr, self.nbytes), "hxa_d2h")
        return out

    def at(self, byte_offset: int) -> int:
        return self.ptr + int(byte_offset)

    def free(self):
        if getattr(self, "ptr", None):
            lib().hxa_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def sync():
    check(lib().hxa_sync(), "hxa_sync")


# ------------------------------------------------------------------------------------------------ packs
LORA_R = 128  # rank of the rapid-moss LoRA of a kind-2 (MOSS + LoRA) pack


def pack_layout(kind: int, D: int, F: int, DC: int, fmt_attn: int, fmt_mlp: int):
    offs = (L * 32)()
    total = lib().hxa_pack_layout(kind, D, F, DC, fmt_attn, fmt_mlp, offs, 32)
    nmat = len(pack_shapes(kind, D, F, DC))
    mats = [(offs[3 * i], offs[3 * i + 1]) for i in range(nmat)]
    return total, mats, offs[3 * nmat]


def pack_shapes(kind: int, D: int, F: int, DC: int):
    """(N, K) of each pack matrix in pack order (kind 0 Anima, 1 MOSS, 2 MOSS with the LoRA columns after K, then
    the four LoRA-A matrices)."""
    if kind == 0:
        return [(3 * D, D), (D, D), (D, D), (2 * D, DC), (D, D), (F, D), (D, F)]
    if kind == 2:
        R = LORA_R
        return [(3 * D, D + 3 * R), (D, D + R), (2 * F, D + R), (D, F + R), (3 * R, D), (R, D), (R, D), (R, F)]
    return [(3 * D, D), (D, D), (2 * F, D), (D, F)]


def pack_fmts(kind: int, fmt_attn: int, fmt_mlp: int):
    """weight format of each pack matrix: attention matrices fmt_attn, MLP ones fmt_mlp"""
    attn = {0: 5, 1: 2, 2: 2}[kind]
    n = len(pack_shapes(kind, 256, 256, 256))
    f = [fmt_attn if i < attn else fmt_mlp for i in range(n)]
    if kind == 2:  # the LoRA-A matrices follow their projections' formats
        f[4], f[5], f[6], f[7] = fmt_attn, fmt_attn, fmt_mlp, fmt_mlp
    return f


def ktile(rows: np.ndarray, N: int, K: int) -> np.ndarray:
    """Bytes of a row-major weight matrix with N rows of 32-deep k groups -> the k-tiled order
    [K/32][N][chunk] (chunk = 64 bytes fp16, 32 q8, 16 q4)."""
    return np.ascontiguousarray(rows.reshape(N, K // 32, -1).transpose(1, 0, 2)).reshape(-1)


def unktile(tiled: np.ndarray, N: int, K: int) -> np.ndarray:
    """Inverse of ktile: k-tiled bytes -> row-major bytes [N][...]."""
    return np.ascontiguousarray(tiled.reshape(K // 32, N, -1).transpose(1, 0, 2)).reshape(-1)


def build_pack(kind: int, D: int, F: int, DC: int, fmt_attn: int, fmt_mlp: int, mats, vec: np.ndarray) -> np.ndarray:
    """Host image of a GPU block pack. mats: per matrix either an fp16 [N][K] array (F16) or a (q, s) pair
    (q8: int8 [N][K]; q4: uint8 [N][K/2]; s: fp16 bits [K/32][N]). vec: the fp32 vector section. The matrices
    are stored k-tiled, the pack layout the block runner reads."""
    total, offs, voff = pack_layout(kind, D, F, DC, fmt_attn, fmt_mlp)
    buf = np.zeros(total, np.uint8)
    shapes = pack_shapes(kind, D, F, DC)
    fmts = pack_fmts(kind, fmt_attn, fmt_mlp)
    assert len(mats) == len(shapes)
    for i, (m, (woff, soff)) in enumerate(zip(mats, offs)):
        fmt = fmts[i]
        N, K = shapes[i]
        if fmt == W_F16:
            a = np.ascontiguousarray(m).view(np.uint8).reshape(-1)
            assert a.size == N * K * 2
            buf[woff:woff + a.size] = ktile(a, N, K)
        else:
            q, s = m
            qa = np.ascontiguousarray(q).view(np.uint8).reshape(-1)
            sa = np.ascontiguousarray(s).view(np.uint8).reshape(-1)
            assert qa.size == (N * K if fmt == W_Q8 else N * K // 2) and sa.size == (K // 32) * N * 2
            buf[woff:woff + qa.size] = ktile(qa, N, K)
            buf[soff:soff + sa.size] = sa
    v = np.ascontiguousarray(vec, np.float32).view(np.uint8).reshape(-1)
    buf[voff:voff + v.size] = v
    return buf


def block_ws(d: BlockDims) -> DeviceArray:
    return DeviceArray((lib().hxa_block_ws_bytes(C.byref(d)),), np.uint8, zero=True)


def ws_buffer(d: BlockDims, ws: DeviceArray, which: int):
    ld = L()
    p = lib().hxa_block_ws_buf(C.byref(d), ws.ptr, which, C.byref(ld))
    return p, ld.value


WS_H, WS_Q, WS_K, WS_VT, WS_O, WS_T1, WS_MID, WS_CK, WS_CVT, WS_T2 = range(10)


def read_ws(d: BlockDims, ws: DeviceArray, which: int, rows: int, cols: int) -> np.ndarray:
    """Copy a stage buffer of the block workspace to host as fp16 [rows][cols] (row stride from the layout)."""
    p, ld = ws_buffer(d, ws, which)
    out = np.zeros((rows, ld), np.float16)
    check(lib().hxa_d2h(out.ctypes.data, p, ((rows - 1) * ld + cols) * 2), "read_ws")
    return np.ascontiguousarray(out[:, :cols])
