"""Pinning the CPU oracle (oracle/hxo.c) before it is trusted as the parity reference.

Every oracle function is checked against something it does not share code with: numpy's IEEE float16
conversion (exhaustively), float64 numpy math (closed forms), brute force, the reference's own integer-hash KAT
generator (hexagon/mega/gtest.c:13, gemm check :34-39), invariants (norm preservation, identity modulation,
masking), and numpy restatements of the reference's own Python layout code (export_block.py:49-54,
export_all.py:7-18, moss/mkblk_test.py:35-39, moss/export_te.py:41-48, moss/moss_ref.py:21-39).
"""
import math

import numpy as np
import pytest

from oracle import hxo


def gen_hash(a, b, s):
    """hexagon/mega/gtest.c:13 gen(a,b,s): integer hash -> value in [-0.5, 0.5) (multiples of 1/256)."""
    a = np.asarray(a, np.uint64)
    b = np.asarray(b, np.uint64)
    h = (a * np.uint64(2654435761) + b * np.uint64(40503) + np.uint64(s)) & np.uint64(0xFFFFFFFF)
    h ^= h >> np.uint64(13)
    h = (h * np.uint64(0x5BD1E995)) & np.uint64(0xFFFFFFFF)
    h ^= h >> np.uint64(15)
    return ((h & np.uint64(255)).astype(np.int64) - 128).astype(np.float32) / 256.0


# ---------------------------------------------------------------------------------------------- fp16
def test_h2f_exhaustive_matches_numpy():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = hxo.h2f(bits)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f2h_matches_numpy_rne():
    rng = np.random.default_rng(0)
    xs = [rng.standard_normal(200000).astype(np.float32) * s for s in (1e-6, 1e-3, 1.0, 100.0, 3e4)]
    # every half value, every midpoint between neighbours (ties), and +-1 float ulp around the midpoints
    h = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mid = ((h[:-1] + h[1:]) / 2).astype(np.float32)
    xs += [mid, np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(0)), -mid]
    xs.append(np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e9, -1e9, np.inf, -np.inf, 2.0**-25, 2.0**-24, 5.96e-8], np.float32))
    x = np.concatenate(xs).astype(np.float32)
    got = hxo.f2h(x)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)
    assert hxo.f2h(np.array([np.nan], np.float32))[0] & 0x7C00 == 0x7C00


# ---------------------------------------------------------------------------------------------- GEMM
@pytest.mark.parametrize("M,N,K", [(64, 96, 128), (37, 53, 300), (96, 256, 512)])
def test_gemm_hash_kat_exact(M, N, K):
    """gtest.c pattern: A = gen(m,k,7), W = gen(k,n,11); values are multiples of 1/256, so the float64
    dot product is exact and the oracle must equal it after one rounding to fp32."""
    m, k = np.meshgrid(np.arange(M), np.arange(K), indexing="ij")
    A = gen_hash(m, k, 7).astype(np.float16)
    k2, n = np.meshgrid(np.arange(K), np.arange(N), indexing="ij")
    Wkn = gen_hash(k2, n, 11).astype(np.float16)
    W = np.ascontiguousarray(Wkn.T)  # [N][K]
    exact = A.astype(np.float64) @ Wkn.astype(np.float64)
    got = hxo.gemm(A, W)
    assert np.array_equal(got, exact.astype(np.float32))
    assert np.array_equal(hxo.gemm(A, W, naive=True), got)


def test_gemm_random_vs_float64():
    rng = np.random.default_rng(1)
    A = rng.standard_normal((130, 1000)).astype(np.float16)
    W = (rng.standard_normal((70, 1000)) * 0.02).astype(np.float16)
    ref = A.astype(np.float64) @ W.astype(np.float64).T
    got = hxo.gemm(A, W)
    assert np.max(np.abs(got - ref) / (np.abs(ref) + 1e-3)) < 1e-6


def test_linear_f32():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((5, 64)).astype(np.float32)
    W = rng.standard_normal((33, 64)).astype(np.float16)
    ref = x.astype(np.float64) @ W.astype(np.float64).T
    assert np.allclose(hxo.linear_f32(x, W), ref, rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------------------------------------- norms
def _ktest_inputs(D=2048, rows=64):
    """hexagon/mega/ktest.c:17-27: LCG s = s*1664525+1013904223, rnd = ((s>>8)&0xFFFF)/32768 - 1;
    x = rnd*300 + 50*(c+cb) per [slab][cb][r][c]; shift = rnd, scale = rnd*0.5."""
    s = 5
    vals = []

    def rnd():
        nonlocal s
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        return ((s >> 8) & 0xFFFF) / 32768.0 - 1.0

    ncb = D // 32
    x = np.zeros((rows, D), np.float32)
    for sl in range(rows // 32):
        for cb in range(ncb):
            for r in range(32):
                for c in range(32):
                    x[sl * 32 + r, cb * 32 + c] = np.float32(rnd() * 300.0 + 50.0 * (c + cb))
    sh = np.zeros(D, np.float32)
    sc = np.zeros(D, np.float32)
    for i in range(D):
        sh[i] = rnd()
        sc[i] = rnd() * 0.5
    return x, sh, sc


def test_lnmod_ktest_vs_double():
    x, sh, sc = _ktest_inputs()
    got = hxo.lnmod(x, sh, sc).view(np.float16).astype(np.float64)
    xd = x.astype(np.float64)
    mu = xd.mean(1, keepdims=True)
    var = (xd * xd).mean(1, keepdims=True) - mu * mu
    ref = (xd - mu) / np.sqrt(var + 1e-6) * (1 + sc.astype(np.float64)) + sh
    ulp = np.abs(ref.astype(np.float16).astype(np.float64) - ref)
    assert np.all(np.abs(got - ref) <= ulp + 1e-12)  # correctly rounded to fp16


def test_lnmod_identity_modulation_normalises():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((16, 512)) * 5 + 3).astype(np.float32)
    h = hxo.lnmod(x, np.zeros(512), np.zeros(512)).view(np.float16).astype(np.float64)
    assert np.all(np.abs(h.mean(1)) < 2e-3)
    assert np.all(np.abs(h.var(1) - 1) < 2e-3)
    # shift/scale act per column as (1+scale)*y + shift
    sh = rng.standard_normal(512).astype(np.float32)
    sc = rng.standard_normal(512).astype(np.float32)
    h2 = hxo.lnmod(x, sh, sc).view(np.float16).astype(np.float64)
    assert np.allclose(h2, h * (1 + sc) + sh, atol=2e-2, rtol=2e-3)


def test_rmsmod_vs_moss_ref_formula():
    """moss_ref.py:21-22 rms(x, w) = x * rsqrt(mean(x^2) + 1e-6) * w, then * (1 + scale) + shift (:61)."""
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((8, 384)) * 20).astype(np.float32)
    w, sh, sc = (rng.standard_normal(384).astype(np.float32) for _ in range(3))
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd * xd).mean(1, keepdims=True) + 1e-6) * w * (1 + sc) + sh
    got = hxo.rmsmod(x, w, sh, sc).view(np.float16).astype(np.float64)
    assert np.allclose(got, ref, rtol=1.5e-3, atol=1e-3)


# ---------------------------------------------------------------------------------------------- RMS + RoPE
def test_rope_pairs_d_with_d_plus_64_rotating_by_plus_theta():
    """kern.c:186-191: x[d] -> x[d] c - x[d+64] s, x[d+64] -> x[d] s + x[d+64] c. A unit vector e_d must land on
    (cos, sin) at (d, d+64) and nowhere else; e_{d+64} on (-sin, cos)."""
    T, D = 64, 256
    ang = np.linspace(0.1, 2.9, T * 64).reshape(T, 64)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    rng = np.random.default_rng(5)
    d = rng.integers(0, 64, T)
    q = np.zeros((T, D), np.float16)
    q[np.arange(T), d] = 1.0  # head 0: unit vector e_d; RMS of e_d = 1/sqrt(128)
    q[np.arange(T), 128 + d + 64] = 1.0  # head 1: e_{d+64}
    got = hxo.rmsrope(q, np.ones(128, np.float32), cos, sin).view(np.float16).astype(np.float64)
    r = math.sqrt(128.0)  # rsqrt(1/128 + eps) ~ sqrt(128)
    c, s = cos[np.arange(T), d], sin[np.arange(T), d]
    assert np.allclose(got[np.arange(T), d], r * c, rtol=2e-3, atol=2e-2)
    assert np.allclose(got[np.arange(T), d + 64], r * s, rtol=2e-3, atol=2e-2)
    assert np.allclose(got[np.arange(T), 128 + d], -r * s, rtol=2e-3, atol=2e-2)
    assert np.allclose(got[np.arange(T), 128 + d + 64], r * c, rtol=2e-3, atol=2e-2)
    mask = np.ones((T, D), bool)
    mask[np.arange(T), d] = mask[np.arange(T), d + 64] = False
    mask[np.arange(T), 128 + d] = mask[np.arange(T), 128 + d + 64] = False
    assert np.all(got[mask] == 0)


def test_rmsrope_norm_and_gain():
    rng = np.random.default_rng(6)
    T, D = 32, 512
    q = (rng.standard_normal((T, D)) * 3).astype(np.float16)
    g = rng.uniform(0.5, 2, 128).astype(np.float32)
    n0 = hxo.rmsrope(q, np.ones(128, np.float32)).view(np.float16).astype(np.float64)
    # RMS-normalised heads have mean square 1
    assert np.allclose((n0.reshape(T, 4, 128) ** 2).mean(-1), 1.0, atol=3e-3)
    ng = hxo.rmsrope(q, g).view(np.float16).astype(np.float64)
    assert np.allclose(ng, (n0.reshape(T, 4, 128) * g).reshape(T, D), rtol=2e-3, atol=2e-3)
    # rotation preserves each (d, d+64) pair norm
    ang = rng.uniform(-7, 7, (T, 64))
    nr = hxo.rmsrope(q, g, np.cos(ang), np.sin(ang)).view(np.float16).astype(np.float64).reshape(T, 4, 2, 64)
    ng4 = ng.reshape(T, 4, 2, 64)
    assert np.allclose((nr ** 2).sum(2), (ng4 ** 2).sum(2), rtol=4e-3, atol=4e-3)


# ---------------------------------------------------------------------------------------------- attention
def _attn_f64(q, k, v, nvalid):
    T, D = q.shape
    out = np.zeros((T, D))
    for h in range(D // 128):
        sl = slice(h * 128, (h + 1) * 128)
        S = q[:, sl].astype(np.float64) @ k[:nvalid, sl].astype(np.float64).T
        P = np.exp(S - S.max(1, keepdims=True))
        out[:, sl] = (P / P.sum(1, keepdims=True)) @ v[:nvalid, sl].astype(np.float64)
    return out


@pytest.mark.parametrize("T,NKV,nvalid", [(96, 96, 96), (64, 160, 150), (32, 64, 33)])
def test_attention_modes_vs_float64_softmax(T, NKV, nvalid):
    rng = np.random.default_rng(7)
    D = 256
    q = (rng.standard_normal((T, D)) * 0.25).astype(np.float16)
    k = rng.standard_normal((NKV, D)).astype(np.float16)
    v = rng.standard_normal((NKV, D)).astype(np.float16)
    ref = _attn_f64(q, k, v, nvalid)
    exact = hxo.attention(q, k, v, nvalid, mode=1).view(np.float16).astype(np.float64)
    assert np.max(np.abs(exact - ref)) < 2e-3
    refr = hxo.attention(q, k, v, nvalid, mode=0).view(np.float16).astype(np.float64)
    assert np.max(np.abs(refr - ref)) < 2e-2  # fp16 S/P/rowsum rounding of the reference
    assert np.linalg.norm(refr - ref) / np.linalg.norm(ref) < 5e-3


def test_attention_special_cases():
    rng = np.random.default_rng(8)
    T, NKV, D = 32, 64, 128
    q = rng.standard_normal((T, D)).astype(np.float16)
    v = rng.standard_normal((NKV, D)).astype(np.float16)
    # identical keys -> uniform weights -> every output row is the mean of V
    k = np.tile(rng.standard_normal((1, D)).astype(np.float16), (NKV, 1))
    for mode in (0, 1):
        o = hxo.attention(q, k, v, mode=mode).view(np.float16).astype(np.float64)
        assert np.allclose(o, v.astype(np.float64).mean(0)[None, :], atol=4e-3)
    # one key aligned with every query and huge -> output = that key's value row
    k2 = np.zeros((NKV, D), np.float16)
    q2 = np.zeros((T, D), np.float16)
    q2[:, 0] = 8.0
    k2[17, 0] = 8.0
    for mode in (0, 1):
        o = hxo.attention(q2, k2, v, mode=mode).view(np.float16)
        assert np.array_equal(o, np.tile(v[17:18], (T, 1)))
    # masked keys (>= nvalid) do not influence the result whatever they hold
    k3 = rng.standard_normal((NKV, D)).astype(np.float16)
    a = hxo.attention(q, k3, v, nvalid=40)
    k3[40:] = 50.0
    v2 = v.copy()
    v2[40:] = 1000.0
    b = hxo.attention(q, k3, v2, nvalid=40)
    assert np.array_equal(a, b)


# ---------------------------------------------------------------------------------------------- activations
def _all_finite_halves():
    b = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = b.view(np.float16)
    return b[np.isfinite(f)]


def test_gelu_erf_table_semantics_exhaustive():
    b = _all_finite_halves()
    x = b.view(np.float16).astype(np.float64)
    got = hxo.gelu(b, 0).view(np.float16).astype(np.float64)
    from scipy.special import erf
    ref = 0.5 * x * (1 + erf(x / math.sqrt(2)))
    # two fp16 roundings (table entry + final subtraction): error <= ~1 ulp of max(|x|, |ref|) scale
    tol = np.maximum(np.abs(x), np.abs(ref)) * 2.0 ** -10 + 2.0 ** -24
    assert np.all(np.abs(got - ref) <= tol)
    for xv, r in ((0.0, 0.0), (1.0, 0.8413447460685429), (-1.0, -0.15865525393145707), (3.0, 2.995950)):
        assert abs(hxo.gelu(np.array([xv], np.float16), 0).view(np.float16)[0] - r) < 2e-3


def test_gelu_tanh_exhaustive():
    b = _all_finite_halves()
    x = b.view(np.float16).astype(np.float64)
    got = hxo.gelu(b, 1).view(np.float16)
    ref = (0.5 * x * (1 + np.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))).astype(np.float16)
    big = np.abs(x) > 10  # x**3 overflow region: both saturate to x or 0
    assert np.array_equal(got[~big].view(np.uint16), ref[~big].view(np.uint16))


def test_situ_vs_moss_ref_formula():
    """moss_ref.py:24-25 situ(h, g) = (4 tanh(g/4) sigmoid(g)) * (25 tanh(h/25)), through the three fp16 tables."""
    rng = np.random.default_rng(9)
    u = (rng.standard_normal(100000) * 10).astype(np.float16)
    g = (rng.standard_normal(100000) * 6).astype(np.float16)
    got = hxo.situ(u, g).view(np.float16).astype(np.float64)
    ud, gd = u.astype(np.float64), g.astype(np.float64)
    ref = 4 * np.tanh(gd / 4) / (1 + np.exp(-gd)) * 25 * np.tanh(ud / 25)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 3 * 2.0 ** -11 + 2.0 ** -20)


def test_resadd_and_split_resadd():
    rng = np.random.default_rng(10)
    x = rng.standard_normal((8, 64)).astype(np.float32)
    t1 = rng.standard_normal((8, 64)).astype(np.float16)
    t2 = rng.standard_normal((8, 64)).astype(np.float16)
    g = rng.standard_normal(64).astype(np.float32)
    assert np.allclose(hxo.resadd(x, t1, g), x + g * t1.astype(np.float32), rtol=1e-6, atol=1e-6)
    assert np.allclose(hxo.resadd2(x, t1, t2, g), x + g * (t1.astype(np.float32) + t2.astype(np.float32)), rtol=1e-6, atol=1e-6)
    assert np.array_equal(hxo.resadd(x, t1, np.zeros(64)), x)  # gate 0: x unchanged


# ---------------------------------------------------------------------------------------------- quantisation
def _q8tiles_ref(w_kn16):
    """numpy restatement of export_all.py:7-18 (wt16 + q8tiles, the 6.2e-5 floor of moss/export_all_q8.py:13)."""
    K, N = w_kn16.shape
    t = np.ascontiguousarray(w_kn16.reshape(K // 32, 16, 2, N // 32, 32).transpose(3, 0, 1, 4, 2))
    a = t.astype(np.float32)
    nb, kb = a.shape[:2]
    s = np.abs(a).max(axis=(2, 4)) / 127.0
    s = np.where(s < 6.2e-5, 6.2e-5, s).astype(np.float16)
    sf = s.astype(np.float32)
    q = np.clip(np.rint(a / sf[:, :, None, :, None]), -127, 127).astype(np.int8)
    q = (q.astype(np.int16) + 128).astype(np.uint8)
    sv = np.repeat(s, 2, axis=2)
    rec = np.concatenate([sv.view(np.uint8).reshape(nb, kb, 128), q.reshape(nb, kb, 1024).view(np.uint8)], axis=2)
    return np.ascontiguousarray(rec).reshape(-1)


def _unpack_q8_ref(rec, nb, kb):
    """numpy restatement of moss/mkblk_test.py:35-39 -> [K, N] float32."""
    r = np.frombuffer(rec.tobytes(), dtype=np.uint8).reshape(nb, kb, 1152)
    sc = r[:, :, :128].copy().view(np.float16)[:, :, 0::2].astype(np.float32)
    q = (r[:, :, 128:].astype(np.int16) - 128).reshape(nb, kb, 16, 32, 2).astype(np.float32) * sc[:, :, None, :, None]
    return q.transpose(1, 2, 4, 0, 3).reshape(kb * 32, nb * 32)


def test_q8_record_matches_reference_packer_and_native_layout():
    rng = np.random.default_rng(11)
    N, K = 96, 128
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    W[3, :32] = 0.0  # an all-zero group exercises the scale floor
    w16 = W.astype(np.float16)
    rec = hxo.q8rec_pack(w16, floor_mode=1)
    assert np.array_equal(rec, _q8tiles_ref(np.ascontiguousarray(w16.T)))
    deq_ref = _unpack_q8_ref(rec, N // 32, K // 32).T  # [N][K]
    deq = hxo.q8rec_unpack(rec, N, K).view(np.float16)
    assert np.array_equal(deq, deq_ref.astype(np.float16))
    # GPU-native layout: same quantiser, same values
    q, s = hxo.q8_quantize(W)
    assert np.array_equal(hxo.q8_dequant(q, s), deq.view(np.uint16))
    assert np.all(np.abs(q.astype(np.int32)) <= 127)
    # value = f16(q*s) exactly, and the quantisation error is within half a step
    sf = s.view(np.float16).astype(np.float32)
    step = np.repeat(sf, 32, axis=0).T  # [N][K]
    d32 = deq.astype(np.float32)
    assert np.all(np.abs(d32 - w16.astype(np.float32)) <= step * 0.5 + np.abs(d32) * 2.0 ** -11 + 1e-7)


def test_q8_exact_for_representable_values():
    rng = np.random.default_rng(12)
    N, K = 64, 64
    qv = rng.integers(-127, 128, (N, K)).astype(np.int8)
    qv[:, ::32] = 127  # every group reaches the max so the derived scale is exactly s
    s = np.float16(0.02 / 127)
    W = (qv.astype(np.float32) * np.float32(s)).astype(np.float16).astype(np.float32)
    q, sc = hxo.q8_quantize(W)
    assert np.all(sc.view(np.float16) == s)
    assert np.array_equal(q, qv)


def _unpack_q4a_ref(rec, nb, kb):
    """numpy restatement of moss/export_te.py:41-48 -> [K, N] float32."""
    r = np.frombuffer(rec.tobytes(), dtype=np.uint8).reshape(nb, kb, 768)
    s = r[:, :, :128].copy().view(np.float16)[:, :, 0::2].astype(np.float32)
    m = r[:, :, 128:256].copy().view(np.float16)[:, :, 0::2].astype(np.float32)
    nib = r[:, :, 256:].reshape(nb, kb, 4, 128)
    v = np.zeros((nb, kb, 4, 2, 128), np.float32)
    v[:, :, :, 0] = nib & 15
    v[:, :, :, 1] = nib >> 4
    v = v.reshape(nb, kb, 16, 32, 2) * s[:, :, None, :, None] + m[:, :, None, :, None]
    return v.transpose(1, 2, 4, 0, 3).reshape(kb * 32, nb * 32)


def test_q4a_record_unpack_matches_reference():
    rng = np.random.default_rng(13)
    N, K = 64, 96
    rec = rng.integers(0, 256, (N // 32) * (K // 32) * 768).astype(np.uint8)
    # sane scales / mins in the two 128 B vectors of each record
    r3 = rec.reshape(-1, 768)
    sv = (rng.uniform(0.001, 0.01, (r3.shape[0], 32))).astype(np.float16)
    mv = (rng.uniform(-0.1, 0.0, (r3.shape[0], 32))).astype(np.float16)
    r3[:, :128] = np.repeat(sv, 2, axis=1).view(np.uint8)
    r3[:, 128:256] = np.repeat(mv, 2, axis=1).view(np.uint8)
    ref = _unpack_q4a_ref(r3.reshape(-1), N // 32, K // 32).T
    got = hxo.q4arec_unpack(r3.reshape(-1), N, K).view(np.float16)
    assert np.array_equal(got, ref.astype(np.float16))


def test_q4_symmetric_roundtrip_and_nibble_order():
    rng = np.random.default_rng(14)
    N, K = 32, 64
    qv = rng.integers(-7, 8, (N, K))  # |q| <= 7 with a 7 in every group: the derived scale is exactly s
    qv[:, ::32] = 7
    s = np.float16(0.02 / 127)
    W = (qv * np.float32(s)).astype(np.float32)
    q, sc = hxo.q4_quantize(W)
    assert np.all(sc.view(np.float16) == s)
    words = q.view(np.uint32).reshape(N, K // 8)
    for k in range(K):
        j = k % 8
        shift = 16 + 4 * (j // 2) if j % 2 else 4 * (j // 2)
        assert np.array_equal(((words[:, k // 8] >> shift) & 15).astype(np.int64) - 8, qv[:, k])
    deq = hxo.q4_dequant(q, sc).view(np.float16).astype(np.float32)
    assert np.array_equal(deq, (qv * np.float32(s)).astype(np.float16).astype(np.float32))
    # asymmetric form value = nibble*s + z reduces to the symmetric one for z = -8 s
    z = (np.full_like(sc.view(np.float16), -8 * s.astype(np.float32))).view(np.uint16)
    assert np.array_equal(hxo.q4_dequant(q, sc, z), hxo.q4_dequant(q, sc))


# ---------------------------------------------------------------------------------------------- tiles
def test_tile_layouts_match_reference_numpy():
    rng = np.random.default_rng(15)
    R, Cc = 64, 96
    a = rng.standard_normal((R, Cc)).astype(np.float16)
    act16 = np.ascontiguousarray(a.reshape(R // 32, 16, 2, Cc // 32, 32).transpose(0, 3, 1, 4, 2)).reshape(-1)  # export_block.py:49-50
    t = hxo.h16_tile(a)
    assert np.array_equal(t, act16.view(np.uint16))
    assert np.array_equal(hxo.h16_untile(t, R, Cc), a.view(np.uint16))
    x = rng.standard_normal((R, Cc)).astype(np.float32)
    x32 = np.ascontiguousarray(x.reshape(R // 32, 32, Cc // 32, 32).transpose(0, 2, 1, 3)).reshape(-1)  # export_block.py:51-52
    assert np.array_equal(hxo.x32_tile(x), x32)
    assert np.array_equal(hxo.x32_untile(x32, R, Cc), x)
    W = rng.standard_normal((Cc, R)).astype(np.float16)  # W[N][K] with N=96, K=64
    wkn = np.ascontiguousarray(W.T)
    wt16 = np.ascontiguousarray(wkn.reshape(R // 32, 16, 2, Cc // 32, 32).transpose(3, 0, 1, 4, 2)).reshape(-1)  # export_all.py:7-8
    assert np.array_equal(hxo.wt16_pack(W), wt16.view(np.uint16))
    assert np.array_equal(hxo.wt16_unpack(wt16.view(np.uint16), Cc, R), W.view(np.uint16))


# ---------------------------------------------------------------------------------------------- RoPE tables
def test_rope_anima_table_closed_form():
    """megarun.cpp:77-90: dim_h = 42, 22 zero (t) angles, then 21 h-frequencies and 21 w-frequencies 10000^(-2i/42)."""
    gh, gw = 6, 5
    c, s = hxo.rope_anima(gh, gw)
    tk = np.arange(gh * gw)
    hh, ww = tk // gw, tk % gw
    f = 1.0 / 10000.0 ** (2.0 * np.arange(21) / 42)
    ang = np.concatenate([np.zeros((gh * gw, 22)), hh[:, None] * f[None], ww[:, None] * f[None]], 1)
    assert np.allclose(c, np.cos(ang), atol=1e-7) and np.allclose(s, np.sin(ang), atol=1e-7)
    assert np.all(c[:, :22] == 1) and np.all(s[:, :22] == 0)


def test_rope_moss_table_vs_moss_ref():
    """numpy restatement of moss_ref.py:27-35 (rope_tables) for a synthetic band vector."""
    H, W, T = 4, 6, 5
    bands = (1.0 / 10000.0 ** (np.arange(16) / 16)).astype(np.float32)
    h, w = np.meshgrid(np.arange(H), np.arange(W), indexing="ij")
    img = np.stack((np.zeros_like(h), np.full_like(h, T), h, w), -1).reshape(-1, 4).astype(np.float64)
    img[:, 2] -= (H - 1) / 2
    img[:, 3] -= (W - 1) / 2
    txt = np.zeros((T, 4))
    txt[:, 1] = np.arange(T)
    phase = np.concatenate((img, txt), 0)[:, :, None] * bands.astype(np.float64)  # [N,4,16]
    r = np.concatenate((np.sin(phase), np.cos(phase)), -2).reshape(len(phase), -1)  # [N,128]
    sin_ref, cos_ref = r[:, :64], r[:, 64:]
    c, s = hxo.rope_moss(H, W, T, bands)
    assert np.allclose(c, cos_ref, atol=1e-6) and np.allclose(s, sin_ref, atol=1e-6)


# ---------------------------------------------------------------------------------------------- glue
def test_patchify_roundtrip_and_order():
    rng = np.random.default_rng(16)
    lat = rng.standard_normal((16, 8, 6)).astype(np.float32)
    tok = hxo.patchify(lat)
    # animad.cpp:447-450: token (gy, gx), feature c*4 + a*2 + b = lat[c][2gy+a][2gx+b]
    assert tok[1 * 3 + 2, 5 * 4 + 1 * 2 + 0] == lat[5, 2 * 1 + 1, 2 * 2 + 0]
    # unpatchify uses feature order (a, b, c) (animad.cpp:490-491)
    y = np.ascontiguousarray(tok.reshape(-1, 16, 2, 2).transpose(0, 2, 3, 1).reshape(-1, 64))
    assert np.array_equal(hxo.unpatchify(y, 16, 8, 6), lat)


def test_sinusoid_and_final_norm():
    s = hxo.sinusoid(0.75, 256)
    i = np.arange(128)
    a = 0.75 * np.exp(-np.log(10000.0) * i / 128)
    assert np.allclose(s[:128], np.cos(a), atol=1e-6) and np.allclose(s[128:], np.sin(a), atol=1e-6)
    rng = np.random.default_rng(17)
    x = (rng.standard_normal((4, 256)) * 3 + 1).astype(np.float32)
    sh, sc = rng.standard_normal(256).astype(np.float32), rng.standard_normal(256).astype(np.float32)
    y = hxo.final_norm(x, sh, sc)
    xd = x.astype(np.float64)
    ref = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-6) * (1 + sc) + sh
    assert np.allclose(y, ref, rtol=1e-5, atol=1e-5)
