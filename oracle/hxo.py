"""ctypes wrapper around the C oracle (oracle/hxo.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the
checker. The product (hexanima_amd/) never imports it.

Arrays are numpy: fp16 tensors are passed as uint16 bit patterns (``x.view(np.uint16)``), fp32 as float32.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libhxo.so")
_lib = None

P = C.c_void_p
I = C.c_int
L = C.c_long


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc, OpenMP)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE] + (["-B"] if force else []), check=True)
    return _LIB_PATH


def use_native() -> str:
    """Build the oracle for this host's CPU (-march=native) and load that copy instead of the portable one; must be
    called before the first oracle call. Returns the compiler command line used."""
    global _LIB_PATH
    if _lib is not None:
        raise RuntimeError("the oracle is already loaded")
    subprocess.run(["make", "-s", "-B", "-C", _HERE, "native"], check=True)
    _LIB_PATH = os.path.join(_HERE, "_build", "libhxo_native.so")
    return subprocess.run(["make", "-s", "-C", _HERE, "native-flags"], check=True, capture_output=True,
                          text=True).stdout.strip()


class _Cfg(C.Structure):
    _fields_ = [("T", I), ("D", I), ("H", I), ("C", I), ("DC", I), ("F", I), ("gelu", I), ("stop", I), ("attn_mode", I)]


class _AW(C.Structure):
    _fields_ = [(n, P) for n in ("wq", "wk", "wv", "wo", "wcq", "wck", "wcv", "wco", "w1", "w2", "gain")]


class _AB(C.Structure):
    _fields_ = [(n, P) for n in ("h", "q", "k", "v", "o", "t", "mid", "ck", "cv")]


class _MCfg(C.Structure):
    _fields_ = [("T", I), ("nvalid", I), ("D", I), ("H", I), ("F", I), ("stop", I), ("attn_mode", I)]


class _MW(C.Structure):
    _fields_ = [(n, P) for n in ("wq", "wk", "wv", "wo", "wup", "wgate", "wdown", "gq", "gk", "n1", "n2", "aqkv", "ao",
                                 "aug", "adn")]


class _MB(C.Structure):
    _fields_ = [(n, P) for n in ("h", "q", "k", "v", "o", "t", "up", "gate", "mid", "lqkv", "lo", "lu", "ld")]


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.endswith("libhxo_native.so"):
            build()
        lb = C.CDLL(_LIB_PATH)
        sig = {
            "hxo_f2h": (C.c_uint16, [C.c_float]),
            "hxo_h2f": (C.c_float, [C.c_uint16]),
            "hxo_f2h_n": (None, [P, P, C.c_size_t]),
            "hxo_h2f_n": (None, [P, P, C.c_size_t]),
            "hxo_set_threads": (I, [I]),
            "hxo_gemm": (None, [P, L, P, L, P, L, I, I, I]),
            "hxo_gemm_naive": (None, [P, L, P, L, P, L, I, I, I]),
            "hxo_linear_f32": (None, [P, L, P, L, P, L, I, I, I]),
            "hxo_lnmod": (None, [P, I, I, P, P, C.c_float, P]),
            "hxo_rmsmod": (None, [P, I, I, P, P, P, C.c_float, P]),
            "hxo_rmsrope": (None, [P, I, L, I, P, P, P, I]),
            "hxo_attention": (None, [P, L, P, L, P, L, P, L, I, I, I, I, I]),
            "hxo_gelu_erf_h": (C.c_uint16, [C.c_uint16]),
            "hxo_gelu_tanh_h": (C.c_uint16, [C.c_uint16]),
            "hxo_situ_h": (C.c_uint16, [C.c_uint16, C.c_uint16]),
            "hxo_gelu_n": (None, [P, C.c_size_t, I]),
            "hxo_situ_n": (None, [P, P, P, C.c_size_t]),
            "hxo_resadd": (None, [P, I, I, P, P]),
            "hxo_resadd2": (None, [P, I, I, P, P, P]),
            "hxo_q8_quantize": (None, [P, I, I, P, P]),
            "hxo_q8_dequant": (None, [P, P, I, I, P]),
            "hxo_q4_quantize": (None, [P, I, I, P, P]),
            "hxo_q4_dequant": (None, [P, P, P, I, I, P]),
            "hxo_h16_tile": (None, [P, I, I, P]),
            "hxo_h16_untile": (None, [P, I, I, P]),
            "hxo_x32_tile": (None, [P, I, I, P]),
            "hxo_x32_untile": (None, [P, I, I, P]),
            "hxo_wt16_pack": (None, [P, I, I, P]),
            "hxo_wt16_unpack": (None, [P, I, I, P]),
            "hxo_q8rec_pack": (None, [P, I, I, P, I]),
            "hxo_q8rec_unpack": (None, [P, I, I, P]),
            "hxo_q4arec_unpack": (None, [P, I, I, P]),
            "hxo_rope_anima": (None, [I, I, P, P]),
            "hxo_rope_moss": (None, [I, I, I, P, P, P]),
            "hxo_rope_moss_scaled": (None, [I, I, I, P, C.c_double, P, P]),
            "hxo_lowres_pool": (None, [P, P, I, I, I, I, C.c_float, P]),
            "hxo_lowres_velocity": (None, [P, P, P, P, I, I, I, I, C.c_float, C.c_double, P, P]),
            "hxo_moss_pool2": (None, [P, I, I, I, P]),
            "hxo_upsample2_rows": (None, [P, I, I, I, P]),
            "hxo_anima_block": (I, [C.POINTER(_Cfg), C.POINTER(_AW), P, P, P, P, P, C.POINTER(_AB)]),
            "hxo_moss_block": (I, [C.POINTER(_MCfg), C.POINTER(_MW), P, P, P, P, C.POINTER(_MB)]),
            "hxo_sinusoid": (None, [C.c_float, I, P]),
            "hxo_patchify": (None, [P, I, I, I, P]),
            "hxo_unpatchify": (None, [P, I, I, I, P]),
            "hxo_final_norm": (None, [P, I, I, P, P]),
        }
        for name, (res, args) in sig.items():
            f = getattr(lb, name)
            f.restype = res
            f.argtypes = args
        _lib = lb
    return _lib


def _p(a) -> int:
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _u16(a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        return a.view(np.uint16)
    assert a.dtype == np.uint16, a.dtype
    return a


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def set_threads(n: int = 0) -> int:
    return lib().hxo_set_threads(n)


def f2h(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().hxo_f2h_n(_p(x), _p(out), x.size)
    return out


def h2f(h) -> np.ndarray:
    h = _u16(h)
    out = np.empty(h.shape, np.float32)
    lib().hxo_h2f_n(_p(h), _p(out), h.size)
    return out


def gemm(A, W, naive: bool = False) -> np.ndarray:
    """C[M][N] = A[M][K] . W[N][K]^T, fp16 operands (uint16 bits), double accumulation, fp32 result."""
    A, W = _u16(A), _u16(W)
    M, K = A.shape
    N, K2 = W.shape
    assert K == K2
    Cm = np.empty((M, N), np.float32)
    fn = lib().hxo_gemm_naive if naive else lib().hxo_gemm
    fn(_p(A), K, _p(W), K, _p(Cm), N, M, N, K)
    return Cm


def linear_f32(x, W) -> np.ndarray:
    x, W = _f32(x), _u16(W)
    M, K = x.shape
    N = W.shape[0]
    y = np.empty((M, N), np.float32)
    lib().hxo_linear_f32(_p(x), K, _p(W), K, _p(y), N, M, N, K)
    return y


def lnmod(x, shift, scale, eps=1e-6) -> np.ndarray:
    x = _f32(x)
    T, D = x.shape
    h = np.empty((T, D), np.uint16)
    shift, scale = _f32(shift), _f32(scale)
    lib().hxo_lnmod(_p(x), T, D, _p(shift), _p(scale), eps, _p(h))
    return h


def rmsmod(x, w, shift, scale, eps=1e-6) -> np.ndarray:
    x = _f32(x)
    T, D = x.shape
    h = np.empty((T, D), np.uint16)
    w, shift, scale = _f32(w), _f32(shift), _f32(scale)
    lib().hxo_rmsmod(_p(x), T, D, _p(w), _p(shift), _p(scale), eps, _p(h))
    return h


def rmsrope(q, gain, cos=None, sin=None) -> np.ndarray:
    q = _u16(q).copy()
    T, D = q.shape
    rope = cos is not None
    c = _f32(cos) if rope else None
    s = _f32(sin) if rope else None
    gain = _f32(gain)
    lib().hxo_rmsrope(_p(q), T, D, D // 128, _p(gain), _p(c), _p(s), int(rope))
    return q


def attention(q, k, v, nvalid=None, mode: int = 0) -> np.ndarray:
    q, k, v = _u16(q), _u16(k), _u16(v)
    T, D = q.shape
    NKV = k.shape[0]
    o = np.empty((T, D), np.uint16)
    lib().hxo_attention(_p(q), D, _p(k), D, _p(v), D, _p(o), D, T, NKV, NKV if nvalid is None else nvalid, D // 128, mode)
    return o


def gelu(t, mode: int) -> np.ndarray:
    t = _u16(t).copy()
    lib().hxo_gelu_n(_p(t), t.size, mode)
    return t


def situ(up, gate) -> np.ndarray:
    up, gate = _u16(up), _u16(gate)
    out = np.empty(up.shape, np.uint16)
    lib().hxo_situ_n(_p(up), _p(gate), _p(out), up.size)
    return out


def resadd(x, t, gate) -> np.ndarray:
    x = _f32(x).copy()
    T, D = x.shape
    t, gate = _u16(t), _f32(gate)
    lib().hxo_resadd(_p(x), T, D, _p(t), _p(gate))
    return x


def resadd2(x, t1, t2, gate) -> np.ndarray:
    x = _f32(x).copy()
    T, D = x.shape
    t1, t2, gate = _u16(t1), _u16(t2), _f32(gate)
    lib().hxo_resadd2(_p(x), T, D, _p(t1), _p(t2), _p(gate))
    return x


def q8_quantize(W):
    W = _f32(W)
    N, K = W.shape
    q = np.empty((N, K), np.int8)
    s = np.empty((K // 32, N), np.uint16)
    lib().hxo_q8_quantize(_p(W), N, K, _p(q), _p(s))
    return q, s


def q8_dequant(q, s) -> np.ndarray:
    q = np.ascontiguousarray(q, np.int8)
    N, K = q.shape
    w = np.empty((N, K), np.uint16)
    s = _u16(s)
    lib().hxo_q8_dequant(_p(q), _p(s), N, K, _p(w))
    return w


def q4_quantize(W):
    W = _f32(W)
    N, K = W.shape
    q = np.empty((N, K // 2), np.uint8)
    s = np.empty((K // 32, N), np.uint16)
    lib().hxo_q4_quantize(_p(W), N, K, _p(q), _p(s))
    return q, s


def q4_dequant(q, s, z=None) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint8)
    N, K2 = q.shape
    K = K2 * 2
    w = np.empty((N, K), np.uint16)
    s = _u16(s)
    z = _u16(z) if z is not None else None
    lib().hxo_q4_dequant(_p(q), _p(s), _p(z), N, K, _p(w))
    return w


def h16_tile(a):
    a = _u16(a)
    R, Cc = a.shape
    t = np.empty(R * Cc, np.uint16)
    lib().hxo_h16_tile(_p(a), R, Cc, _p(t))
    return t


def h16_untile(t, R, Cc):
    a = np.empty((R, Cc), np.uint16)
    t = _u16(t)
    lib().hxo_h16_untile(_p(t), R, Cc, _p(a))
    return a


def x32_tile(a):
    a = _f32(a)
    R, Cc = a.shape
    t = np.empty(R * Cc, np.float32)
    lib().hxo_x32_tile(_p(a), R, Cc, _p(t))
    return t


def x32_untile(t, R, Cc):
    a = np.empty((R, Cc), np.float32)
    t = _f32(t)
    lib().hxo_x32_untile(_p(t), R, Cc, _p(a))
    return a


def wt16_pack(wNK):
    w = _u16(wNK)
    N, K = w.shape
    t = np.empty(N * K, np.uint16)
    lib().hxo_wt16_pack(_p(w), N, K, _p(t))
    return t


def wt16_unpack(t, N, K):
    w = np.empty((N, K), np.uint16)
    t = _u16(t)
    lib().hxo_wt16_unpack(_p(t), N, K, _p(w))
    return w


def q8rec_pack(wNK, floor_mode: int = 1):
    w = _u16(wNK)
    N, K = w.shape
    rec = np.empty((N // 32) * (K // 32) * 1152, np.uint8)
    lib().hxo_q8rec_pack(_p(w), N, K, _p(rec), floor_mode)
    return rec


def q8rec_unpack(rec, N, K):
    w = np.empty((N, K), np.uint16)
    rec = np.ascontiguousarray(rec, np.uint8)
    lib().hxo_q8rec_unpack(_p(rec), N, K, _p(w))
    return w


def q4arec_unpack(rec, N, K):
    w = np.empty((N, K), np.uint16)
    rec = np.ascontiguousarray(rec, np.uint8)
    lib().hxo_q4arec_unpack(_p(rec), N, K, _p(w))
    return w


def rope_anima(gh, gw):
    T = gh * gw
    c = np.empty((T, 64), np.float32)
    s = np.empty((T, 64), np.float32)
    lib().hxo_rope_anima(gh, gw, _p(c), _p(s))
    return c, s


def rope_moss(H, W, ntxt, bands16):
    T = H * W + ntxt
    c = np.empty((T, 64), np.float32)
    s = np.empty((T, 64), np.float32)
    bands16 = _f32(bands16)
    lib().hxo_rope_moss(H, W, ntxt, _p(bands16), _p(c), _p(s))
    return c, s


def rope_moss_scaled(H, W, ntxt, bands16, scale):
    """moss/mossrun/mossrun.cpp:190-201 with image positions times `scale` (the low-res steps, :313)"""
    T = H * W + ntxt
    c = np.empty((T, 64), np.float32)
    s = np.empty((T, 64), np.float32)
    bands16 = _f32(bands16)
    lib().hxo_rope_moss_scaled(H, W, ntxt, _p(bands16), float(scale), _p(c), _p(s))
    return c, s


def lowres_pool(nfull, dhat, f, t):
    """phone/animad.cpp:429-437: [C][H][W] noise and clean estimate -> the [C][H/f][W/f] latent of a 1/f step"""
    nfull, dhat = _f32(nfull), _f32(dhat)
    Cc, H, W = nfull.shape
    out = np.empty((Cc, H // f, W // f), np.float32)
    lib().hxo_lowres_pool(_p(nfull), _p(dhat), Cc, H, W, f, float(t), _p(out))
    return out


def lowres_velocity(xlow, vlow, xfull, nfull, f, t, tn):
    """phone/animad.cpp:486-503: (dhat, v) -- the upsampled clean estimate and the full-res velocity that lands the
    Euler step from t to tn on (1 - tn) dhat + tn noise"""
    xlow, vlow, xfull, nfull = _f32(xlow), _f32(vlow), _f32(xfull), _f32(nfull)
    Cc, H, W = xfull.shape
    dhat = np.empty_like(xfull)
    vf = np.empty_like(xfull)
    lib().hxo_lowres_velocity(_p(xlow), _p(vlow), _p(xfull), _p(nfull), Cc, H, W, f, float(t), float(tn), _p(dhat), _p(vf))
    return dhat, vf


def moss_pool2(z, H, W):
    """moss/mossrun/mossrun.cpp:291: token rows [H*W][C4] -> 2 x the 2x2 mean, [(H/2)*(W/2)][C4]"""
    z = _f32(z)
    out = np.empty(((H // 2) * (W // 2), z.shape[1]), np.float32)
    lib().hxo_moss_pool2(_p(z), H, W, z.shape[1], _p(out))
    return out


def upsample2_rows(src, h, w):
    """moss/mossrun/mossrun.cpp:278-282: token rows [h*w][C4] -> bilinear 2x, [(2h)*(2w)][C4]"""
    src = _f32(src)
    out = np.empty((4 * h * w, src.shape[1]), np.float32)
    lib().hxo_upsample2_rows(_p(src), h, w, src.shape[1], _p(out))
    return out


def sinusoid(t, dim):
    out = np.empty(dim, np.float32)
    lib().hxo_sinusoid(float(t), dim, _p(out))
    return out


def patchify(lat):
    lat = _f32(lat)
    Cc, H, W = lat.shape
    tok = np.empty(((H // 2) * (W // 2), Cc * 4), np.float32)
    lib().hxo_patchify(_p(lat), Cc, H, W, _p(tok))
    return tok


def unpatchify(y, Cc, H, W):
    lat = np.empty((Cc, H, W), np.float32)
    y = _f32(y)
    lib().hxo_unpatchify(_p(y), Cc, H, W, _p(lat))
    return lat


def final_norm(x, shift, scale):
    x = _f32(x).copy()
    T, D = x.shape
    shift, scale = _f32(shift), _f32(scale)
    lib().hxo_final_norm(_p(x), T, D, _p(shift), _p(scale))
    return x


ANIMA_W = ("wq", "wk", "wv", "wo", "wcq", "wck", "wcv", "wco", "w1", "w2")


def anima_block(x, ctx, mod9, cos, sin, w: dict, *, H, F, gelu=1, stop=0, attn_mode=0):
    """One Anima-structure block. x fp32 [T][D] (not modified; the result is returned), ctx fp16 [C][DC],
    mod9 fp32 [9][D], cos/sin [T][64], w: W[N][K] fp16 matrices + gain [4][128].
    Returns (x_out, stage buffers dict, number of stages run)."""
    x = _f32(x).copy()
    T, D = x.shape
    ctx = _u16(ctx)
    Cn, DC = ctx.shape
    ws = {k: _u16(w[k]) for k in ANIMA_W}
    gain = _f32(w["gain"]).reshape(-1)
    buf = {k: np.zeros((T, D), np.uint16) for k in ("h", "q", "k", "v", "o", "t")}
    buf["mid"] = np.zeros((T, F), np.uint16)
    buf["ck"] = np.zeros((Cn, D), np.uint16)
    buf["cv"] = np.zeros((Cn, D), np.uint16)
    cfg = _Cfg(T, D, H, Cn, DC, F, gelu, stop, attn_mode)
    aw = _AW(*[_p(ws[k]) for k in ANIMA_W], _p(gain))
    ab = _AB(*[_p(buf[k]) for k in ("h", "q", "k", "v", "o", "t", "mid", "ck", "cv")])
    mod9 = _f32(mod9)
    cos, sin = _f32(cos), _f32(sin)
    n = lib().hxo_anima_block(C.byref(cfg), C.byref(aw), _p(x), _p(ctx), _p(mod9), _p(cos), _p(sin), C.byref(ab))
    return x, buf, n


MOSS_W = ("wq", "wk", "wv", "wo", "wup", "wgate", "wdown")
MOSS_A = ("aqkv", "ao", "aug", "adn")
LORA_R = 128


def moss_block(x, mod6, cos, sin, w: dict, *, H, F, nvalid=None, stop=0, attn_mode=0):
    """One MOSS-class block. w: fp16 W[N][K] matrices wq, wk, wv, wo, wup, wgate, wdown, the fp32 vectors gq, gk,
    n1, n2 and, for the rapid-moss LoRA (moss/hexagon/mega/blk.c:238-259), the A matrices aqkv [384][D], ao [128][D],
    aug [128][D], adn [128][F] with every W then carrying its 128 scaled B columns after K ([N][K + 128]).
    Returns (x_out, stage buffers dict, number of stages run)."""
    x = _f32(x).copy()
    T, D = x.shape
    lora = w.get("aqkv") is not None
    R = LORA_R if lora else 0
    ws = {k: _u16(w[k]) for k in MOSS_W}
    for k in ("wq", "wk", "wv", "wo"):
        assert ws[k].shape == (D, D + R), (k, ws[k].shape)
    assert ws["wup"].shape == (F, D + R) and ws["wgate"].shape == (F, D + R) and ws["wdown"].shape == (D, F + R)
    aw = {k: _u16(w[k]) for k in MOSS_A} if lora else {}
    vec = {k: _f32(w[k]) for k in ("gq", "gk", "n1", "n2")}
    buf = {k: np.zeros((T, D), np.uint16) for k in ("h", "q", "k", "v", "o", "t")}
    for k in ("up", "gate", "mid"):
        buf[k] = np.zeros((T, F), np.uint16)
    buf["lqkv"] = np.zeros((T, 3 * max(R, 1)), np.uint16)
    for k in ("lo", "lu", "ld"):
        buf[k] = np.zeros((T, max(R, 1)), np.uint16)
    cfg = _MCfg(T, T if nvalid is None else nvalid, D, H, F, stop, attn_mode)
    mw = _MW(*[_p(ws[k]) for k in MOSS_W], *[_p(vec[k]) for k in ("gq", "gk", "n1", "n2")],
             *[_p(aw[k]) if lora else None for k in MOSS_A])
    mb = _MB(*[_p(buf[k]) for k in ("h", "q", "k", "v", "o", "t", "up", "gate", "mid", "lqkv", "lo", "lu", "ld")])
    mod6 = _f32(mod6)
    cos, sin = _f32(cos), _f32(sin)
    n = lib().hxo_moss_block(C.byref(cfg), C.byref(mw), _p(x), _p(mod6), _p(cos), _p(sin), C.byref(mb))
    return x, buf, n
