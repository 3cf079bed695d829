"""GPU parity of the individual HIP kernels against the CPU oracle, through the C-ABI (hexanima_amd/hip.py).

Tolerances (fp16 storage): a GEMM output may differ from the oracle's correctly rounded value by one fp16 ulp plus
the fp32 accumulation-order error 4 sqrt(K) 2^-24 sum|a w| (tests/_helpers.assert_gemm_close), and >= 98% of the
outputs must be bit-identical; norm outputs by at most 1 ulp. Attention uses an fp32 online softmax,
so it is compared with the oracle's exact-softmax mode (max abs 4e-3, rel-l2 1e-3) and with the reference-rounding
mode (rel-l2 4.7e-3, the reference's own fp16 S/P rounding noise), about 3x the measured errors."""
import numpy as np
import pytest

from oracle import hxo
from tests._helpers import assert_gemm_close, f16, rel, ulp_diff

pytestmark = pytest.mark.gpu


def _hip():
    from hexanima_amd import hip
    hip.init()
    return hip


def say(msg):
    print(f"[case] {msg}", flush=True)


# ------------------------------------------------------------------------------------------------ GEMM
def _run_gemm(hip, A, fmt, w, s, N, K, epi=0, ksplit=1, tile=None, x=None, gate=None, z=None):
    M = A.shape[0]
    dA = hip.DeviceArray.from_numpy(f16(A))
    dW = hip.DeviceArray.from_numpy(w)
    dS = hip.DeviceArray.from_numpy(s) if s is not None else None
    dZ = hip.DeviceArray.from_numpy(z) if z is not None else None
    resadd = epi in (hip.EPI_RESADD, hip.EPI_RESADD_SPLIT2)
    if resadd:
        dx = hip.DeviceArray.from_numpy(x.astype(np.float32))
        dg = hip.DeviceArray.from_numpy(gate.astype(np.float32))
        out = None
    elif epi == hip.EPI_PARTIAL:
        out = hip.DeviceArray((ksplit, M, N), np.float16)
    elif epi == hip.EPI_STORE_T:
        out = hip.DeviceArray((N, M), np.float16)
    elif epi == hip.EPI_SITU:
        out = hip.DeviceArray((M, N // 2), np.float16)
    else:
        out = hip.DeviceArray((M, N), np.float16)
    ldo = {hip.EPI_STORE_T: M, hip.EPI_SITU: N // 2}.get(epi, N)
    args = (dA.ptr, K, M, fmt, dW.ptr, dS.ptr if dS else None, dZ.ptr if dZ else None, N, K, ksplit, epi,
            out.ptr if out else None, ldo,
            M * N, dx.ptr if resadd else None, N, dg.ptr if resadd else None)
    if tile:
        hip.check(hip.lib().hxa_gemm_tile(*args, tile[0], tile[1], tile[2] if len(tile) > 2 else 0, None), "gemm_tile")
    else:
        hip.check(hip.lib().hxa_gemm(*args, None, 0, 0, None), "gemm")
    hip.sync()
    return dx.numpy() if resadd else out.numpy()


# waves 9: the ping-pong 8-wave kernel
@pytest.mark.parametrize("tile", [None, (192, 256), (192, 256, 8), (192, 192), (192, 128), (256, 128), (128, 256), (128, 128),
                                  (64, 128), (128, 64), (192, 256, 9), (256, 256, 9), (128, 256, 9), (128, 128, 9)])
def test_gemm_f16_tiles(tile):
    hip = _hip()
    say(f"gemm f16 tile={tile}")
    rng = np.random.default_rng(0)
    M, N, K = 320, 384, 512  # ragged in M for every tile shape
    A = rng.standard_normal((M, K))
    W = f16(rng.standard_normal((N, K)) * 0.05)
    got = _run_gemm(hip, A, 0, W, None, N, K, tile=tile)
    assert_gemm_close(got, hxo.gemm(f16(A), W), f16(A), W)


@pytest.mark.parametrize("N,K", [(6144, 2048), (2048, 2048), (8192, 2048), (2048, 8192)])
@pytest.mark.parametrize("fmt", [1, 2])
def test_gemm_w8a16_w4a16_config1(N, K, fmt):
    """The W8A16 / W4A16 microbench shapes (M = 1536): dequantised-fp16 GEMM is the reference."""
    hip = _hip()
    say(f"gemm fmt={fmt} M=1536 N={N} K={K}")
    rng = np.random.default_rng(N + K + fmt)
    M = 1536
    A = f16(rng.standard_normal((M, K)))
    s = np.full((K // 32, N), np.float16(0.02 / 127)).view(np.uint16)
    if fmt == 1:
        q = rng.integers(-127, 128, (N, K)).astype(np.int8)
        wdq = hxo.q8_dequant(q, s)
    else:
        qv = rng.integers(-8, 8, (N, K))
        q = np.zeros((N, K // 8), np.uint32)
        for j in range(8):
            sh = 16 + 4 * (j // 2) if j % 2 else 4 * (j // 2)
            q |= ((qv[:, j::8] + 8).astype(np.uint32) << sh)
        q = q.view(np.uint8).reshape(N, K // 2)
        wdq = hxo.q4_dequant(q, s)
        assert np.array_equal(wdq.view(np.float16).astype(np.float32), (qv * np.float32(np.float16(0.02 / 127))).astype(np.float16).astype(np.float32))
    got = _run_gemm(hip, A, fmt, q, s, N, K)
    assert_gemm_close(got, hxo.gemm(A, wdq), A, wdq.view(np.float16))


@pytest.mark.parametrize("tile", [(192, 256, 8), (128, 256, 8), (192, 128, 8), (128, 128, 8), (128, 128, 4), (192, 256, 9),
                                  (256, 256, 9), (128, 256, 9), (192, 256, 4), (256, 128, 4), (128, 256, 4), (192, 128, 4),
                                  (192, 192, 4), (64, 128, 4)])
@pytest.mark.parametrize("fmt", [1, 2])
def test_gemm_quant_tiles(fmt, tile):
    """int8 / int4 weights on every 8-wave and 4-wave tile, ragged in M and N (every wave loads its share of the
    scale vectors): dequantised-fp16 GEMM is the reference."""
    hip = _hip()
    say(f"gemm fmt={fmt} tile={tile}")
    rng = np.random.default_rng(40 + fmt)
    M, N, K = 320, 384, 512
    A = f16(rng.standard_normal((M, K)))
    wf = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    q, s = hxo.q8_quantize(wf) if fmt == 1 else hxo.q4_quantize(wf)
    wdq = hxo.q8_dequant(q, s) if fmt == 1 else hxo.q4_dequant(q, s)
    got = _run_gemm(hip, A, fmt, q, s, N, K, tile=tile)
    assert_gemm_close(got, hxo.gemm(A, wdq), A, wdq.view(np.float16))


@pytest.mark.parametrize("tile", [(192, 256, 9), (256, 256, 9), (128, 128, 4), (192, 256, 4), (128, 128, 8)])
@pytest.mark.parametrize("fmt", [1, 2])
def test_gemm_quant_splitk4_partials(fmt, tile):
    """int8 / int4 weights split-K 4 into fp16 partials (the block runner's attention-output / MLP-down form at
    1024 - 4095 rows), including one k step per slice boundary case (K / 4 = 64, two k steps per slice): each partial
    against the oracle's GEMM over its K quarter."""
    hip = _hip()
    say(f"gemm fmt={fmt} split-K 4 partials tile={tile}")
    rng = np.random.default_rng(90 + fmt)
    M, N = 320, 384
    for K in (256, 1024):
        A = f16(rng.standard_normal((M, K)))
        wf = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
        q, s = hxo.q8_quantize(wf) if fmt == 1 else hxo.q4_quantize(wf)
        wdq = hxo.q8_dequant(q, s) if fmt == 1 else hxo.q4_dequant(q, s)
        got = _run_gemm(hip, A, fmt, q, s, N, K, epi=hip.EPI_PARTIAL, ksplit=4, tile=tile)
        for z in range(4):
            sl = slice(z * K // 4, (z + 1) * K // 4)
            Az, Wz = np.ascontiguousarray(A[:, sl]), np.ascontiguousarray(wdq.view(np.float16)[:, sl])
            assert_gemm_close(got[z], hxo.gemm(Az, Wz.view(np.uint16)), Az, Wz)


def _q4a_weights(rng, N, K):
    """Asymmetric int4 (q4a, moss/export_te.py:1-3, dequantised as moss/hexagon/mega/gemm2.c:39-56): nibble in
    [0, 15] with a per-(32-row group, column) fp16 scale s and min z, value f16(nibble * s + z). Packed in the GPU
    order (k0+2j at bits 4j, k0+2j+1 at bits 16+4j of each 32-bit word)."""
    nib = rng.integers(0, 16, (N, K))
    q = np.zeros((N, K // 8), np.uint32)
    for j in range(8):
        sh = 16 + 4 * (j // 2) if j % 2 else 4 * (j // 2)
        q |= nib[:, j::8].astype(np.uint32) << sh
    s = f16(rng.uniform(0.002, 0.01, (K // 32, N)))
    z = f16(-8.0 * s.astype(np.float32) + rng.uniform(-0.01, 0.01, (K // 32, N)))
    return q.view(np.uint8).reshape(N, K // 2), s.view(np.uint16), z.view(np.uint16)


@pytest.mark.parametrize("tile", [None, (128, 128, 4), (192, 256, 4), (128, 256, 8), (192, 256, 9), (128, 256, 9),
                                  (192, 128, 8)])
def test_gemm_q4_asymmetric(tile):
    """q4a weights (a scale and a min per group) through hxa_gemm with z != NULL, ragged in M: the dequantised-fp16
    GEMM is the reference."""
    hip = _hip()
    say(f"gemm q4a tile={tile}")
    rng = np.random.default_rng(77)
    M, N, K = 320, 384, 512
    A = f16(rng.standard_normal((M, K)))
    q, s, z = _q4a_weights(rng, N, K)
    wdq = hxo.q4_dequant(q, s, z)
    got = _run_gemm(hip, A, 2, q, s, N, K, tile=tile, z=z)
    assert_gemm_close(got, hxo.gemm(A, wdq), A, wdq.view(np.float16))


@pytest.mark.parametrize("fmt,asym,ktiled", [(1, False, False), (1, False, True), (2, False, True), (2, True, False),
                                             (2, True, True)])
def test_dequant_pass_equals_oracle_and_fused_gemm(fmt, asym, ktiled):
    """The block runner's dequantisation pass (hxa_dequant): its fp16 output is bit-identical to the oracle's
    f16(q*s) / f16(nibble*s + z) (gemm2.c:19-35, moss gemm2.c:39-56), and an fp16 GEMM on it gives the same bits as
    the fused int8 / int4 GEMM on the same tile (both feed the MFMAs the same values in the same k order)."""
    hip = _hip()
    say(f"dequant pass fmt={fmt} asym={asym} ktiled={ktiled}")
    rng = np.random.default_rng(90 + fmt + 2 * asym)
    M, N, K = 320, 384, 512
    A = f16(rng.standard_normal((M, K)))
    z = None
    if fmt == 1:
        q, s = hxo.q8_quantize((rng.standard_normal((N, K)) * 0.05).astype(np.float32))
        wdq = hxo.q8_dequant(q, s)
    elif asym:
        q, s, z = _q4a_weights(rng, N, K)
        wdq = hxo.q4_dequant(q, s, z)
    else:
        q, s = hxo.q4_quantize((rng.standard_normal((N, K)) * 0.05).astype(np.float32))
        wdq = hxo.q4_dequant(q, s)
    qb = np.ascontiguousarray(q).view(np.uint8).reshape(-1)
    src = hip.ktile(qb, N, K) if ktiled else qb
    fl = fmt | (hip.W_KTILED if ktiled else 0)
    dq_, ds = hip.DeviceArray.from_numpy(src), hip.DeviceArray.from_numpy(s)
    dz = hip.DeviceArray.from_numpy(z) if z is not None else None
    out = hip.DeviceArray((K // 32, N, 32), np.float16)
    hip.check(hip.lib().hxa_dequant(fl, dq_.ptr, ds.ptr, dz.ptr if dz else None, N, K, out.ptr, None), "dequant")
    hip.sync()
    w16 = hip.unktile(out.numpy().view(np.uint8).reshape(-1), N, K).view(np.uint16).reshape(N, K)
    assert np.array_equal(w16, wdq)
    kt16 = out.numpy().reshape(-1)
    for tile in ((128, 128, 4), (192, 256, 8) if fmt == 1 else (128, 256, 8), (192, 256, 9)):
        via_pass = _run_gemm(hip, A, hip.W_F16 | hip.W_KTILED, kt16, None, N, K, tile=tile)
        fused = _run_gemm(hip, A, fl, src, s, N, K, tile=tile, z=z)
        assert np.array_equal(via_pass.view(np.uint16), fused.view(np.uint16)), tile
    assert_gemm_close(via_pass, hxo.gemm(A, wdq), A, wdq.view(np.float16))


def test_gemm_epilogues():
    hip = _hip()
    rng = np.random.default_rng(3)
    M, N, K = 256, 512, 256
    A = f16(rng.standard_normal((M, K)))
    W = f16(rng.standard_normal((N, K)) * 0.1)
    t = f16(hxo.gemm(A, W))

    def t_gpu_for(epi):  # the GPU's own f16(acc) from a plain store on the tile the epilogue launch picks (kernels
        pk = hip.gemm_pick(M, N, K, 0, 1, epi)  # differ in their k order, so f16(acc) may differ by an ulp)
        return _run_gemm(hip, A, 0, W, None, N, K, tile=(pk["bm"], pk["bn"], pk["waves"]))
    say("gemm epi gelu tanh / erf")
    for epi, mode in ((1, 1), (2, 0)):
        got = _run_gemm(hip, A, 0, W, None, N, K, epi=epi)
        ref = hxo.gelu(t_gpu_for(epi), mode).view(np.float16)  # the activation on the same values
        assert ulp_diff(got, ref).max() <= 2
    say("gemm epi store_t")
    got = _run_gemm(hip, A, 0, W, None, N, K, epi=4)
    assert_gemm_close(np.ascontiguousarray(got.T), hxo.gemm(A, W), A, W)
    say("gemm epi resadd")
    x = rng.standard_normal((M, N)).astype(np.float32)
    g = rng.standard_normal(N).astype(np.float32)
    got = _run_gemm(hip, A, 0, W, None, N, K, epi=3, x=x, gate=g)
    # x + g * f16(acc); the f16(acc) may differ by one ulp from the oracle's rounding
    assert np.allclose(got, hxo.resadd(x, t, g), atol=np.abs(g).max() * 2e-3 * np.abs(t.astype(np.float32)).max())
    say("gemm epi partial (split-K 2)")
    got = _run_gemm(hip, A, 0, W, None, N, K, epi=6, ksplit=2)
    for z, sl in ((0, slice(0, K // 2)), (1, slice(K // 2, K))):
        Az, Wz = np.ascontiguousarray(A[:, sl]), np.ascontiguousarray(W[:, sl])
        assert_gemm_close(got[z], hxo.gemm(Az, Wz), Az, Wz)
    say("gemm epi situ (interleaved up/gate)")
    F = N // 2
    up = np.ascontiguousarray(W.reshape(F // 32, 2, 32, K)[:, 0].reshape(F, K))
    gt = np.ascontiguousarray(W.reshape(F // 32, 2, 32, K)[:, 1].reshape(F, K))
    got = _run_gemm(hip, A, 0, W, None, N, K, epi=5)
    t_gpu = t_gpu_for(5)
    tu = np.ascontiguousarray(t_gpu.reshape(M, F // 32, 2, 32)[:, :, 0].reshape(M, F))
    tg = np.ascontiguousarray(t_gpu.reshape(M, F // 32, 2, 32)[:, :, 1].reshape(M, F))
    ref = hxo.situ(tu, tg).view(np.float16)
    assert ulp_diff(got, ref).max() <= 2


def test_gelu_epilogues_every_fp16_input():
    """Both GELU epilogues over every finite fp16 value: with A the identity (K = M = 256) the GEMM's f16(acc) is W^T
    exactly, and W holds each finite fp16 bit pattern once (inf / NaN patterns, which would turn the zero products
    into NaN, and -0 replaced by 0). GELU-erf goes through the epilogue's T2 lookup table; both are checked against the
    oracle's table semantics (kern.c:235-260)."""
    hip = _hip()
    say("gemm GELU epilogues over every finite fp16 input")
    pat = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    pat[((pat & 0x7C00) == 0x7C00) | (pat == 0x8000)] = 0  # inf / NaN, and -0 (the zero products sum to +0)
    W = pat.view(np.float16).reshape(256, 256)
    A = np.eye(256, dtype=np.float16)
    t = np.ascontiguousarray(W.T)
    assert np.array_equal(_run_gemm(hip, A, 0, W, None, 256, 256).view(np.uint16), t.view(np.uint16))
    for epi, mode in ((hip.EPI_GELU_ERF, 0), (hip.EPI_GELU_TANH, 1)):
        got = _run_gemm(hip, A, 0, W, None, 256, 256, epi=epi)
        ref = hxo.gelu(t, mode).view(np.float16)
        d = ulp_diff(got, ref)
        print(f"epi {epi}: max ulp {d.max()}, {int((d > 0).sum())} of {d.size} outputs differ", flush=True)
        assert d.max() <= 2


@pytest.mark.parametrize("fmt,tile", [(f, t) for f in (0, 1, 2)
                                      for t in ((256, 256, 9), (192, 256, 9), (128, 256, 9), (128, 128, 9), (192, 128, 8),
                                                (192, 128, 4))
                                      if not (f == 2 and t == (128, 128, 9))])
def test_gemm_partial_split_k_tiles(fmt, tile):
    """Split-K into two fp16 partials (the K halves of the MLP-down and of the deferred attention-output projection)
    on the ping-pong, 8-wave and 4-wave tiles for each weight format: each half is the oracle GEMM of its K half;
    M and N ragged against the tiles."""
    hip = _hip()
    say(f"gemm partial ksplit=2 fmt={fmt} tile={tile}")
    rng = np.random.default_rng(60 + fmt)
    M, N, K = 320, 416, 1024
    A = f16(rng.standard_normal((M, K)))
    if fmt == 0:
        w, s = f16(rng.standard_normal((N, K)) * 0.05), None
        wd = w.view(np.uint16)
    else:
        wf = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
        w, s = hxo.q8_quantize(wf) if fmt == 1 else hxo.q4_quantize(wf)
        wd = hxo.q8_dequant(w, s) if fmt == 1 else hxo.q4_dequant(w, s)
    got = _run_gemm(hip, A, fmt, w, s, N, K, epi=hip.EPI_PARTIAL, ksplit=2, tile=tile)
    for z, sl in ((0, slice(0, K // 2)), (1, slice(K // 2, K))):
        Az, Wz = np.ascontiguousarray(A[:, sl]), np.ascontiguousarray(wd[:, sl])
        assert_gemm_close(got[z], hxo.gemm(Az, Wz), Az, Wz.view(np.float16))


@pytest.mark.parametrize("fmt,tile", [(0, None), (0, (64, 128)), (1, None), (2, None)])
def test_gemm_resadd_split2_matches_partial_then_resadd2(fmt, tile):
    """The fused split-K residual (blk.c:172-174) equals the two fp16 PARTIAL halves + resadd2, bit for bit, and the
    oracle's resadd2 on those halves."""
    hip = _hip()
    rng = np.random.default_rng(11)
    M, N, K = 320, 256, 1024
    A = f16(rng.standard_normal((M, K)))
    if fmt == 0:
        w, s = f16(rng.standard_normal((N, K)) * 0.05), None
    else:
        wf = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
        w, s = hxo.q8_quantize(wf) if fmt == 1 else hxo.q4_quantize(wf)
    x = rng.standard_normal((M, N)).astype(np.float32)
    g = rng.standard_normal(N).astype(np.float32)
    say(f"gemm resadd_split2 fmt={fmt} tile={tile}")
    got = _run_gemm(hip, A, fmt, w, s, N, K, epi=hip.EPI_RESADD_SPLIT2, x=x, gate=g, tile=tile)
    parts = _run_gemm(hip, A, fmt, w, s, N, K, epi=hip.EPI_PARTIAL, ksplit=2, tile=tile)
    ref = hxo.resadd2(x, parts[0], parts[1], g)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)) or np.abs(got - ref).max() <= 1e-6 * np.abs(ref).max()
    dx = hip.DeviceArray.from_numpy(x)
    dt = [hip.DeviceArray.from_numpy(np.ascontiguousarray(parts[z])) for z in (0, 1)]
    dg = hip.DeviceArray.from_numpy(g)
    hip.check(hip.lib().hxa_resadd2(dx.ptr, N, dt[0].ptr, dt[1].ptr, N, M, N, dg.ptr, None), "resadd2")
    hip.sync()
    assert np.array_equal(got.view(np.uint32), dx.numpy().view(np.uint32))
    # K must split into two halves of whole 64-k step pairs; ksplit must be 1
    bad = _run_gemm_rc(hip, A[:, :96], N, 96, hip.EPI_RESADD_SPLIT2, x, g)
    assert bad == -12


@pytest.mark.parametrize("fmt,tile,epi,ksplit", [(0, None, 0, 1), (0, (192, 256, 8), 0, 1), (0, (64, 128), 0, 1),
                                                (0, None, 6, 2), (1, None, 0, 1), (1, (128, 64), 0, 1), (2, None, 0, 1),
                                                (2, None, 6, 2), (0, None, 7, 1), (1, None, 3, 1), (0, (192, 256, 9), 1, 1),
                                                (0, (192, 256, 9), 6, 2), (0, (128, 128, 9), 3, 1), (0, (256, 256, 9), 0, 1)])
def test_gemm_ktiled_weights_equal_row_major(fmt, tile, epi, ksplit):
    """W stored k-tiled ([K/32][N][chunk], the block-pack layout) gives the same bits as W row-major, for every
    format, tile family and split-K form; N is ragged against the 256-wide tiles."""
    hip = _hip()
    say(f"gemm k-tiled fmt={fmt} tile={tile} epi={epi} ksplit={ksplit}")
    rng = np.random.default_rng(31)
    M, N, K = 320, 416, 1024
    A = f16(rng.standard_normal((M, K)))
    if fmt == 0:
        w, s = f16(rng.standard_normal((N, K)) * 0.05), None
    else:
        wf = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
        w, s = hxo.q8_quantize(wf) if fmt == 1 else hxo.q4_quantize(wf)
    wt = hip.ktile(np.ascontiguousarray(w).view(np.uint8).reshape(-1), N, K)
    assert np.array_equal(hip.unktile(wt, N, K), np.ascontiguousarray(w).view(np.uint8).reshape(-1))
    x = rng.standard_normal((M, N)).astype(np.float32)
    g = rng.standard_normal(N).astype(np.float32)
    kw = dict(epi=epi, ksplit=ksplit, tile=tile, x=x, gate=g)
    ref = _run_gemm(hip, A, fmt, w, s, N, K, **kw)
    got = _run_gemm(hip, A, fmt | hip.W_KTILED, wt, s, N, K, **kw)
    assert np.array_equal(got.view(np.uint8), ref.view(np.uint8))


def _run_gemm_rc(hip, A, N, K, epi, x, g):
    dA = hip.DeviceArray.from_numpy(f16(A))
    dW = hip.DeviceArray((N, K), np.float16)
    dx = hip.DeviceArray.from_numpy(x)
    dg = hip.DeviceArray.from_numpy(g)
    return hip.lib().hxa_gemm(dA.ptr, K, A.shape[0], 0, dW.ptr, None, None, N, K, 1, epi, None, N, 0, dx.ptr, N, dg.ptr,
                              None, 0, 0, None)


@pytest.mark.parametrize("M", [256, 300])
def test_gemm_fused_qkv_split_transposed(M):
    """q|k row-major and v transposed from one projection; M = 300 leaves a partial 8-row run in the transposed
    store (rows past M are not written)."""
    hip = _hip()
    say(f"gemm fused qkv with transposed v M={M}")
    rng = np.random.default_rng(4)
    D = 256
    ldt = (M + 7) // 8 * 8
    A = f16(rng.standard_normal((M, D)))
    W = f16(rng.standard_normal((3 * D, D)) * 0.05)
    dA, dW = hip.DeviceArray.from_numpy(A), hip.DeviceArray.from_numpy(W)
    qk = hip.DeviceArray((M, 2 * D), np.float16)
    vt = hip.DeviceArray.from_numpy(np.full((D, ldt), 7.0, np.float16))
    hip.check(hip.lib().hxa_gemm(dA.ptr, D, M, 0, dW.ptr, None, None, 3 * D, D, 1, 0, qk.ptr, 2 * D, 0, None, 0, None,
                                 vt.ptr, ldt, 2 * D, None), "qkv")
    hip.sync()
    ref = hxo.gemm(A, W)
    Wq, Wv = np.ascontiguousarray(W[:2 * D]), np.ascontiguousarray(W[2 * D:])
    assert_gemm_close(qk.numpy(), ref[:, :2 * D], A, Wq)
    got_t = vt.numpy()
    assert_gemm_close(np.ascontiguousarray(got_t[:, :M].T), ref[:, 2 * D:], A, Wv)
    assert (got_t[:, M:] == 7.0).all()


@pytest.mark.parametrize("rope,fmt", [(True, 0), (False, 0), (True, 1)])
def test_gemm_headnorm_equals_gemm_then_rmsrope(rope, fmt):
    """The projection with the per-head RMSNorm (+ RoPE) fused into its store (kern.c:163-197 in the GEMM flush)
    equals the plain projection followed by the standalone RMS+RoPE kernel, bit for bit; q and k take their own
    gains, the v columns go transposed and un-normalised. Two images of 128 tokens share the RoPE table."""
    hip = _hip()
    say(f"gemm headnorm rope={rope} fmt={fmt}")
    rng = np.random.default_rng(21)
    T, D, B = 128, 256, 2
    M = B * T
    A = f16(rng.standard_normal((M, D)))
    if fmt == 0:
        W, S = f16(rng.standard_normal((3 * D, D)) * 0.05), None
    else:
        W, S = hxo.q8_quantize((rng.standard_normal((3 * D, D)) * 0.05).astype(np.float32))
    gq = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    gk = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    cos, sin = hxo.rope_anima(8, 16)
    dA, dW = hip.DeviceArray.from_numpy(A), hip.DeviceArray.from_numpy(W)
    dS = hip.DeviceArray.from_numpy(S) if S is not None else None
    dq, dk = hip.DeviceArray.from_numpy(gq), hip.DeviceArray.from_numpy(gk)
    dc, ds = hip.DeviceArray.from_numpy(cos), hip.DeviceArray.from_numpy(sin)
    qk = hip.DeviceArray((M, 2 * D), np.float16)
    vt = hip.DeviceArray((D, M), np.float16)
    hip.check(hip.lib().hxa_gemm_headnorm(dA.ptr, D, M, fmt, dW.ptr, dS.ptr if dS else None, None, 3 * D, D, qk.ptr, 2 * D,
                                          vt.ptr, M, 2 * D, 2 * D, dq.ptr, dk.ptr, D, dc.ptr if rope else None,
                                          ds.ptr if rope else None, T, None), "gemm_headnorm")
    qk2 = hip.DeviceArray((M, 2 * D), np.float16)
    vt2 = hip.DeviceArray((D, M), np.float16)
    hip.check(hip.lib().hxa_gemm(dA.ptr, D, M, fmt, dW.ptr, dS.ptr if dS else None, None, 3 * D, D, 1, 0, qk2.ptr, 2 * D, 0,
                                 None, 0, None, vt2.ptr, M, 2 * D, None), "gemm")
    hip.sync()
    plain = qk2.numpy()  # the projection before the head norm
    hip.check(hip.lib().hxa_rmsrope(qk2.ptr, qk2.ptr + 2 * D, dq.ptr, dk.ptr, 2 * D, M, D // 128, dc.ptr if rope else None,
                                    ds.ptr if rope else None, T, None), "rmsrope")
    hip.sync()
    assert np.array_equal(qk.numpy().view(np.uint16), qk2.numpy().view(np.uint16))
    assert np.array_equal(vt.numpy().view(np.uint16), vt2.numpy().view(np.uint16))
    # and against the oracle's RMS+RoPE of the GPU's own projection
    ref = plain
    for part, g in ((slice(0, D), gq), (slice(D, 2 * D), gk)):
        for b in range(B):
            rows = slice(b * T, (b + 1) * T)
            o = hxo.rmsrope(np.ascontiguousarray(ref[rows, part]), g, cos if rope else None, sin if rope else None)
            assert ulp_diff(qk.numpy()[rows, part], o.view(np.float16)).max() <= 1


def test_gemm_rejects_bad_shapes():
    hip = _hip()
    say("gemm argument checks")
    dA = hip.DeviceArray((64, 96), np.float16, zero=True)
    dW = hip.DeviceArray((64, 96), np.float16, zero=True)
    out = hip.DeviceArray((64, 64), np.float16)
    rc = hip.lib().hxa_gemm(dA.ptr, 96, 64, 0, dW.ptr, None, None, 64, 80, 1, 0, out.ptr, 64, 0, None, 0, None, None, 0, 0, None)
    assert rc == -12  # K % 32 != 0
    rc = hip.lib().hxa_gemm(dA.ptr, 96, 64, 0, dW.ptr, None, None, 64, 96, 2, 6, out.ptr, 64, 0, None, 0, None, None, 0, 0, None)
    assert rc == -12  # K / ksplit % 32 != 0
    rc = hip.lib().hxa_gemm(dA.ptr, 96, 64, 1, dW.ptr, None, None, 64, 64, 1, 0, out.ptr, 64, 0, None, 0, None, None, 0, 0, None)
    assert rc == -12  # q8 without scales


# ------------------------------------------------------------------------------------------------ attention
def test_attention_rejects_bad_strides():
    """Row pitches whose per-lane tile offsets would not fit 31 bits, and NKV not a multiple of 8, are argument errors
    (-12) reported before any launch."""
    hip = _hip()
    say("attention argument checks")
    d = hip.DeviceArray((64, 128), np.float16, zero=True)
    L = hip.lib()
    assert L.hxa_attention(d.ptr, 128, d.ptr, 1 << 24, d.ptr, 64, d.ptr, 128, 64, 64, 64, 1, 1, 0, 0, 0, 0, None) == -12
    assert L.hxa_attention(d.ptr, 128, d.ptr, 128, d.ptr, 1 << 23, d.ptr, 128, 64, 64, 64, 1, 1, 0, 0, 0, 0, None) == -12
    assert L.hxa_attention(d.ptr, 128, d.ptr, 128, d.ptr, 64, d.ptr, 128, 64, 60, 60, 1, 1, 0, 0, 0, 0, None) == -12


def _attn(hip, q, k, v, nvalid=None, batch=1):
    T, D = q.shape[0] // batch, q.shape[1]
    NKV = k.shape[0] // batch
    H = D // 128
    dq, dk = hip.DeviceArray.from_numpy(f16(q)), hip.DeviceArray.from_numpy(f16(k))
    vt = np.ascontiguousarray(f16(v).T)  # [D][batch*NKV]
    dv = hip.DeviceArray.from_numpy(vt)
    do = hip.DeviceArray((batch * T, D), np.float16)
    hip.check(hip.lib().hxa_attention(dq.ptr, D, dk.ptr, D, dv.ptr, batch * NKV, do.ptr, D, T, NKV,
                                      NKV if nvalid is None else nvalid, H, batch, T * D, NKV * D, NKV, T * D, None), "attn")
    hip.sync()
    return do.numpy()


# 128-query workgroups (8 waves); odd tile counts (448 keys: 7, 520 valid of 576: 9) leave the second key half one
# tile short
# the last case is the MOSS-class joint attention at its own shape (6144 image + 512 text tokens, 24 heads); the
# oracle (rows are independent) is evaluated on a sample of 416 query rows spread over all key tiles' range.
# Whole key tiles in a multiple of 4 (1536, 6656, 1024 over 1000 ragged queries, and 512 over 200) take the
# ping-pong form: the key halves one phase apart; 320 keys on 5 tiles and 384 keys on 6 do not qualify
@pytest.mark.parametrize("T,NKV,nvalid,H", [(1536, 1536, 1536, 16), (1536, 256, 256, 16), (448, 448, 430, 4), (96, 64, 64, 2),
                                            (1024, 1024, 1000, 32), (300, 512, 500, 3), (200, 576, 520, 2),
                                            (200, 512, 512, 3), (96, 320, 320, 2), (6656, 6656, 6656, 24),
                                            (1000, 1024, 1024, 4), (384, 384, 384, 2)])
def test_attention_vs_oracle(T, NKV, nvalid, H):
    hip = _hip()
    say(f"attention T={T} NKV={NKV} nvalid={nvalid} H={H}")
    rng = np.random.default_rng(T + NKV)
    D = 128 * H
    # unit-RMS q/k heads with the 1/sqrt(128) gain folded into q, as after the RMS+RoPE stage
    q = f16(rng.standard_normal((T, D)) / np.sqrt(128) * 2.0)
    k = f16(rng.standard_normal((NKV, D)))
    v = f16(rng.standard_normal((NKV, D)))
    got = _attn(hip, q, k, v, nvalid).astype(np.float64)
    rows = np.arange(T) if T * NKV * H <= 64 << 20 else np.unique(np.r_[np.arange(0, T, 16), T - 1])
    got = got[rows]
    exact = hxo.attention(q[rows], k, v, nvalid, mode=1).view(np.float16).astype(np.float64)
    refr = hxo.attention(q[rows], k, v, nvalid, mode=0).view(np.float16).astype(np.float64)
    mx, r1, r0 = np.max(np.abs(got - exact)), rel(got, exact), rel(got, refr)
    print(f"attention rows={rows.size}: max abs {mx:.2e}, rel vs exact {r1:.2e}, rel vs reference rounding {r0:.2e}",
          flush=True)
    assert mx < 4e-3  # measured 9.8e-4 - 2.0e-3 (one or two fp16 ulps of outputs near 1)
    assert r1 < 1e-3  # measured 2.1e-4 - 3.2e-4
    assert r0 < 4.7e-3  # measured 8.2e-4 - 1.6e-3


# (M, T, NKV, nvalid): the 2B block's cross site (1536 tokens, 256 text tokens); batch 2 of 256 tokens over 77 of 80
# text keys (ragged, the last tile masked); three key tiles, the third ragged (190 of 200); megarun's 512 context
# tokens (more than four key tiles: the online form)
@pytest.mark.parametrize("M,T,NKV,nvalid", [(1536, 1536, 256, 256), (512, 256, 80, 77), (256, 256, 200, 190),
                                            (384, 384, 512, 512)])
def test_cross_attention_fused_vs_oracle(M, T, NKV, nvalid):
    """hxa_cross_attention_fused: the cross-q projection with its per-head RMSNorm * gain and the attention of every
    head over its image's text keys in one kernel, against the oracle's GEMM (fp16 store), rmsrope (no RoPE) and
    exact-softmax attention, image by image; and against the unfused GPU path (head-norm GEMM, attention kernel)."""
    hip = _hip()
    say(f"fused cross attention M={M} T={T} NKV={NKV} nvalid={nvalid}")
    L = hip.lib()
    rng = np.random.default_rng(M + NKV)
    D, H = 2048, 16
    B = M // T
    h = f16(rng.standard_normal((M, D)))
    W = f16(rng.standard_normal((D, D)) * 0.02)
    gain = (np.full(128, 128 ** -0.5) * rng.uniform(0.8, 1.2, 128)).astype(np.float32)
    k = f16(rng.standard_normal((B * NKV, D)))
    v = f16(rng.standard_normal((B * NKV, D)))
    dh, dW, dg, dk = (hip.DeviceArray.from_numpy(a) for a in (h, W, gain, k))
    dvt = hip.DeviceArray.from_numpy(np.ascontiguousarray(v.T))  # [D][B * NKV]
    do = hip.DeviceArray((M, D), np.float16)
    hip.check(L.hxa_cross_attention_fused(dh.ptr, D, M, T, 0, dW.ptr, D, D, dg.ptr, dk.ptr, D, dvt.ptr, B * NKV, NKV, nvalid,
                                          NKV * D, NKV, do.ptr, D, None), "cross_attention_fused")
    hip.sync()
    got = do.numpy().astype(np.float64)
    # q = f16(RMSNorm(f16(h W^T)) * gain) per head (the projection's fp16 store, then the head norm)
    q16 = hxo.rmsrope(f16(hxo.gemm(h, W)).view(np.uint16), gain).view(np.float16)
    ref = np.concatenate([hxo.attention(q16[b * T:(b + 1) * T], k[b * NKV:(b + 1) * NKV], v[b * NKV:(b + 1) * NKV], nvalid,
                                        mode=1).view(np.float16) for b in range(B)]).astype(np.float64)
    mx, r = float(np.max(np.abs(got - ref))), rel(got, ref)
    # the unfused GPU path: hxa_gemm_headnorm (no RoPE) into q, then hxa_attention
    dq = hip.DeviceArray((M, D), np.float16)
    hip.check(L.hxa_gemm_headnorm(dh.ptr, D, M, 0, dW.ptr, None, None, D, D, dq.ptr, D, None, 0, D, D, dg.ptr, dg.ptr, D,
                                  None, None, 0, None), "gemm_headnorm")
    du = hip.DeviceArray((M, D), np.float16)
    hip.check(L.hxa_attention(dq.ptr, D, dk.ptr, D, dvt.ptr, B * NKV, du.ptr, D, T, NKV, nvalid, H, B, T * D, NKV * D, NKV,
                              T * D, None), "attention")
    hip.sync()
    mu = float(np.max(np.abs(got - du.numpy().astype(np.float64))))
    print(f"fused cross attention: max abs {mx:.2e}, rel vs exact {r:.2e}; max abs vs unfused GPU path {mu:.2e}", flush=True)
    assert mx < 4e-3 and r < 1e-3  # the attention kernel's bounds (test_attention_vs_oracle)
    assert mu < 2e-3


def test_cross_attention_fused_rejects_unfit_shapes():
    hip = _hip()
    L = hip.lib()
    buf = hip.DeviceArray((4 << 20,), np.uint8)
    g = hip.DeviceArray((128,), np.float32)
    # T not a multiple of 128, int8 weights: argument errors, nothing launched
    assert L.hxa_cross_attention_fused(buf.ptr, 2048, 320, 160, 0, buf.ptr, 2048, 2048, g.ptr, buf.ptr, 2048, buf.ptr, 256,
                                       256, 256, 0, 0, buf.ptr, 2048, None) == -12
    assert L.hxa_cross_attention_fused(buf.ptr, 2048, 256, 256, 1, buf.ptr, 2048, 2048, g.ptr, buf.ptr, 2048, buf.ptr, 256,
                                       256, 256, 0, 0, buf.ptr, 2048, None) == -12


def test_clock_record_gemm_and_attention():
    """hxa_clock_record: one record per workgroup with a plausible shader clock, results unchanged, and nothing
    written once it is switched off."""
    hip = _hip()
    say("clock record: 1536 x 2048 x 2048 GEMM (128 workgroups or more), 1536 x 1536 attention, 16 heads")
    L = hip.lib()
    rng = np.random.default_rng(5)
    A = f16(rng.standard_normal((1536, 2048)))
    W = f16(rng.standard_normal((2048, 2048)) * 0.02)
    plain = _run_gemm(hip, A, 0, W, None, 2048, 2048)
    recs = [hip.DeviceArray((4096 * 4,), np.uint64, zero=True) for _ in range(2)]
    for kind, r in enumerate(recs):
        hip.check(L.hxa_clock_record(kind, r.ptr, 4096), "clock_record")
    try:
        timed = _run_gemm(hip, A, 0, W, None, 2048, 2048)
        q = f16(rng.standard_normal((1536, 2048)) / np.sqrt(128))
        k, v = f16(rng.standard_normal((1536, 2048))), f16(rng.standard_normal((1536, 2048)))
        _attn(hip, q, k, v)
    finally:
        for kind in range(2):
            hip.check(L.hxa_clock_record(kind, None, 0), "clock_record")
    assert np.array_equal(plain.view(np.uint16), timed.view(np.uint16))
    pk = hip.gemm_pick(1536, 2048, 2048, 0)
    nwg_gemm = -(-1536 // pk["bm"]) * -(-2048 // pk["bn"])
    for r, nwg in ((recs[0], nwg_gemm), (recs[1], None)):
        b = r.numpy().reshape(4096, 4).astype(np.float64)
        ok = b[:, 3] > b[:, 1]
        if nwg is not None:
            assert ok[:nwg].all() and not ok[nwg:].any()
        assert ok.sum() >= 128
        ghz = (b[ok, 2] - b[ok, 0]) / (b[ok, 3] - b[ok, 1]) * 0.1
        print(f"clock record: {ok.sum()} workgroups, {ghz.min():.2f} - {ghz.max():.2f} GHz", flush=True)
        assert (ghz > 0.3).all() and (ghz < 3.5).all()
    # switched off: a further launch leaves the (cleared) records alone
    hip.check(L.hxa_memset(recs[0].ptr, 0, recs[0].nbytes), "memset")
    _run_gemm(hip, A, 0, W, None, 2048, 2048)
    assert not recs[0].numpy().any()


def test_attention_batched_images_are_independent():
    hip = _hip()
    say("attention batch=3")
    rng = np.random.default_rng(9)
    T, NKV, D = 128, 96, 256
    q = f16(rng.standard_normal((3 * T, D)) * 0.2)
    k = f16(rng.standard_normal((3 * NKV, D)))
    v = f16(rng.standard_normal((3 * NKV, D)))
    got = _attn(hip, q, k, v, batch=3)
    for b in range(3):
        one = _attn(hip, q[b * T:(b + 1) * T], k[b * NKV:(b + 1) * NKV], v[b * NKV:(b + 1) * NKV])
        assert np.array_equal(got[b * T:(b + 1) * T], one)


# ------------------------------------------------------------------------------------------------ elementwise
@pytest.mark.parametrize("D", [2048, 2560, 3072])
@pytest.mark.parametrize("rms", [False, True])
def test_norm_mod(D, rms):
    hip = _hip()
    say(f"norm_mod D={D} rms={rms}")
    rng = np.random.default_rng(D)
    T = 96
    x = (rng.standard_normal((T, D)) * 3 + 0.5).astype(np.float32)
    sh, sc, w = (rng.standard_normal(D).astype(np.float32) * 0.3 for _ in range(3))
    dx, dsh, dsc, dw = (hip.DeviceArray.from_numpy(a) for a in (x, sh, sc, w))
    h = hip.DeviceArray((T, D), np.float16)
    hip.check(hip.lib().hxa_norm_mod(dx.ptr, D, T, D, dsh.ptr, dsc.ptr, dw.ptr if rms else None, 1e-6, h.ptr, D, None), "norm")
    hip.sync()
    ref = hxo.rmsmod(x, w, sh, sc) if rms else hxo.lnmod(x, sh, sc)
    assert ulp_diff(h.numpy(), ref.view(np.float16)).max() <= 1


@pytest.mark.parametrize("rope", [False, True])
def test_rmsrope(rope):
    hip = _hip()
    say(f"rmsrope rope={rope}")
    rng = np.random.default_rng(11)
    T, D = 256, 512
    q = f16(rng.standard_normal((T, D)) * 2)
    g = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    cos, sin = hxo.rope_anima(16, 16)
    dq = hip.DeviceArray.from_numpy(q)
    dg = hip.DeviceArray.from_numpy(g)
    dc, ds = hip.DeviceArray.from_numpy(cos), hip.DeviceArray.from_numpy(sin)
    hip.check(hip.lib().hxa_rmsrope(dq.ptr, None, dg.ptr, None, D, T, D // 128, dc.ptr if rope else None,
                                    ds.ptr if rope else None, T, None), "rmsrope")
    hip.sync()
    ref = hxo.rmsrope(q, g, cos if rope else None, sin if rope else None).view(np.float16)
    assert ulp_diff(dq.numpy(), ref).max() <= 1


@pytest.mark.parametrize("rms", [False, True])
def test_resadd_norm_mod_equals_resadd_then_norm(rms):
    """The previous site's gated residual applied inside the next site's norm kernel equals the residual update
    followed by the norm, bit for bit (x and h)."""
    hip = _hip()
    say(f"resadd + norm_mod rms={rms}")
    rng = np.random.default_rng(13)
    T, D = 96, 2048
    x = rng.standard_normal((T, D)).astype(np.float32)
    t = f16(rng.standard_normal((T, D)))
    g, sh, sc = (rng.standard_normal(D).astype(np.float32) * 0.5 for _ in range(3))
    w = rng.uniform(0.5, 1.5, D).astype(np.float32)
    dx1, dx2 = hip.DeviceArray.from_numpy(x), hip.DeviceArray.from_numpy(x)
    dt, dz = hip.DeviceArray.from_numpy(t), hip.DeviceArray((T, D), np.float16, zero=True)
    dg, dsh, dsc, dw = (hip.DeviceArray.from_numpy(a) for a in (g, sh, sc, w))
    h1, h2 = hip.DeviceArray((T, D), np.float16), hip.DeviceArray((T, D), np.float16)
    wp = dw.ptr if rms else None
    hip.check(hip.lib().hxa_resadd_norm_mod(dx1.ptr, D, T, D, dt.ptr, D, dg.ptr, dsh.ptr, dsc.ptr, wp, 1e-6, h1.ptr, D, None),
              "resadd_norm_mod")
    hip.check(hip.lib().hxa_resadd2(dx2.ptr, D, dt.ptr, dz.ptr, D, T, D, dg.ptr, None), "resadd2")
    hip.check(hip.lib().hxa_norm_mod(dx2.ptr, D, T, D, dsh.ptr, dsc.ptr, wp, 1e-6, h2.ptr, D, None), "norm_mod")
    hip.sync()
    assert np.array_equal(dx1.numpy().view(np.uint32), dx2.numpy().view(np.uint32))
    assert np.array_equal(h1.numpy().view(np.uint16), h2.numpy().view(np.uint16))
    assert np.array_equal(dx1.numpy(), hxo.resadd(x, t, g))


def test_resadd2_and_tile_conversions():
    hip = _hip()
    say("resadd2 + x32 conversions")
    rng = np.random.default_rng(12)
    T, D = 64, 256
    x = rng.standard_normal((T, D)).astype(np.float32)
    t1, t2 = f16(rng.standard_normal((T, D))), f16(rng.standard_normal((T, D)))
    g = rng.standard_normal(D).astype(np.float32)
    dx, d1, d2, dg = (hip.DeviceArray.from_numpy(a) for a in (x, t1, t2, g))
    hip.check(hip.lib().hxa_resadd2(dx.ptr, D, d1.ptr, d2.ptr, D, T, D, dg.ptr, None), "resadd2")
    hip.sync()
    assert np.array_equal(dx.numpy(), hxo.resadd2(x, t1, t2, g))
    tiles = hxo.x32_tile(x)
    dt = hip.DeviceArray.from_numpy(tiles)
    rows = hip.DeviceArray((T, D), np.float32)
    hip.check(hip.lib().hxa_x32_to_rows(dt.ptr, rows.ptr, T, D, None), "x32_to_rows")
    back = hip.DeviceArray((T * D,), np.float32)
    hip.check(hip.lib().hxa_rows_to_x32(rows.ptr, back.ptr, T, D, None), "rows_to_x32")
    hip.sync()
    assert np.array_equal(rows.numpy(), x) and np.array_equal(back.numpy(), tiles)


def test_quantize_matches_oracle():
    hip = _hip()
    say("quantize q8 / q4")
    rng = np.random.default_rng(13)
    N, K = 96, 256
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    W[5, :32] = 0
    dW = hip.DeviceArray.from_numpy(W)
    for fmt, (qo, so) in ((1, hxo.q8_quantize(W)), (2, hxo.q4_quantize(W))):
        q = hip.DeviceArray(qo.shape, qo.dtype)
        s = hip.DeviceArray(so.shape, np.uint16)
        hip.check(hip.lib().hxa_quantize(dW.ptr, N, K, fmt, q.ptr, s.ptr, None), "quantize")
        hip.sync()
        assert np.array_equal(s.numpy(), so) and np.array_equal(q.numpy(), qo)
        # k-tiled output: the same bytes in [K/32][N][chunk] order, scales unchanged
        hip.check(hip.lib().hxa_quantize(dW.ptr, N, K, fmt | hip.W_KTILED, q.ptr, s.ptr, None), "quantize k-tiled")
        hip.sync()
        assert np.array_equal(s.numpy(), so)
        assert np.array_equal(q.numpy().view(np.uint8).reshape(-1), hip.ktile(qo.view(np.uint8).reshape(-1), N, K))


@pytest.mark.parametrize("M,N,K,fmt,ksplit,epi,norm", [(1536, 8192, 2048, 0, 1, 1, 0), (1536, 6144, 2048, 0, 1, 0, 4096),
                                                       (1536, 10240, 2560, 1, 1, 1, 0), (320, 384, 512, 2, 2, 6, 0),
                                                       (256, 4096, 1024, 1, 1, 0, 0)])
def test_gemm_pick_names_the_tile_hxa_gemm_runs(M, N, K, fmt, ksplit, epi, norm):
    """hxa_gemm_pick reports the tile hxa_gemm runs: forcing that tile gives the same bits as the automatic choice;
    the pick respects head-norm (whole heads per tile) and int4 (bn >= 128) limits; bad sizes give hxa_gemm's error."""
    hip = _hip()
    say(f"gemm_pick M={M} N={N} K={K} fmt={fmt} ksplit={ksplit} epi={epi} norm={norm}")
    pk = hip.gemm_pick(M, N, K, fmt, ksplit, epi, norm)
    assert pk["waves"] in (4, 8, 9) and pk["rounds"] >= 1
    assert pk["rounds"] == -(-(-(-M // pk["bm"]) * -(-N // pk["bn"]) * ksplit) // hip.device_info()["num_cu"])
    if norm:
        assert pk["bn"] % 128 == 0 and norm % pk["bn"] == 0
    if fmt == 2:
        assert pk["bn"] >= 128
    if norm:
        return  # hxa_gemm_headnorm's pick; the plain-store comparison below does not apply
    rng = np.random.default_rng(70)
    Mt = min(M, 512)
    A = f16(rng.standard_normal((Mt, K)))
    if fmt == 0:
        w, s = f16(rng.standard_normal((N, K)) * 0.05), None
    else:
        wf = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
        w, s = hxo.q8_quantize(wf) if fmt == 1 else hxo.q4_quantize(wf)
    pk_t = hip.gemm_pick(Mt, N, K, fmt, ksplit, epi, 0)
    auto = _run_gemm(hip, A, fmt, w, s, N, K, epi=epi, ksplit=ksplit)
    forced = _run_gemm(hip, A, fmt, w, s, N, K, epi=epi, ksplit=ksplit, tile=(pk_t["bm"], pk_t["bn"], pk_t["waves"]))
    assert np.array_equal(auto.view(np.uint16), forced.view(np.uint16))
    with pytest.raises(RuntimeError):
        hip.gemm_pick(M, N, K + 16, fmt, ksplit, epi, 0)


@pytest.mark.parametrize("fmt,tile", [(2, (128, 128, 9)), (0, (96, 128, 4)), (0, (192, 256, 5)), (1, (256, 128, 8)),
                                      (2, (128, 64, 4)), (0, (256, 256, 4))])
def test_gemm_forced_tile_without_kernel_is_an_argument_error(fmt, tile):
    """A forced tile with no kernel for that shape / wave count / format is rejected with HXA_E_ARG (-12) before
    anything is launched."""
    hip = _hip()
    say(f"gemm forced tile {tile} fmt={fmt}")
    M, N, K = 256, 256, 256
    dA = hip.DeviceArray((M, K), np.float16, zero=True)
    dW = hip.DeviceArray((N * K,), np.float16, zero=True)
    dS = hip.DeviceArray((K // 32 * N,), np.float16, zero=True)
    out = hip.DeviceArray((M, N), np.float16)
    rc = hip.lib().hxa_gemm_tile(dA.ptr, K, M, fmt, dW.ptr, dS.ptr if fmt else None, None, N, K, 1, 0, out.ptr, N, 0,
                                 None, 0, None, tile[0], tile[1], tile[2], None)
    assert rc == -12


# ------------------------------------------------------------------------------------------------ split-K linear
def test_sum_partials_exact():
    """hxa_sum_partials: fp32 slices added in slice order and rounded once to fp16, bit for bit with numpy's float32
    sums; row padding (ldp > N, ldo > N) read and left alone."""
    hip = _hip()
    rng = np.random.default_rng(7)
    M, N, ldp, ldo = 37, 72, 80, 88
    for S in (1, 2, 3, 4):
        say(f"sum_partials S={S}")
        p = (rng.standard_normal((S, M, ldp)) * 3.0).astype(np.float32)
        ref = p[0, :, :N].copy()
        for z in range(1, S):
            ref = (ref + p[z, :, :N]).astype(np.float32)
        dp = hip.DeviceArray.from_numpy(p)
        out0 = np.full((M, ldo), np.float16(-7.0))
        dout = hip.DeviceArray.from_numpy(out0)
        hip.check(hip.lib().hxa_sum_partials(dp.ptr, S, M * ldp, ldp, M, N, dout.ptr, ldo, None), "sum_partials")
        hip.sync()
        got = dout.numpy()
        assert np.array_equal(got[:, :N].view(np.uint16), ref.astype(np.float16).view(np.uint16))
        assert np.all(got[:, N:] == np.float16(-7.0))


@pytest.mark.parametrize("fmt,tile", [(f, t) for f in (0, 1, 2)
                                      for t in (None, (128, 128, 4), (192, 128, 4), (128, 256, 8), (192, 256, 9),
                                                (128, 128, 9))
                                      if not (f == 2 and t == (128, 128, 9))])  # (no int4 ping-pong 128x128 kernel)
def test_gemm_partial_f32_slices(fmt, tile):
    """PARTIAL_F32: each of 4 K slices' fp32 sums (no fp16 rounding) against the oracle's double-accumulated GEMM
    over that slice, within the fp32 accumulation bound 4 sqrt(K/4) 2^-24 sum|a w| + 2^-24 |ref|; ragged M and N."""
    hip = _hip()
    say(f"gemm PARTIAL_F32 fmt={fmt} tile={tile}")
    rng = np.random.default_rng(120 + fmt)
    M, N, K, S = 320, 392, 1024, 4
    A = f16(rng.standard_normal((M, K)))
    wf = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    if fmt == 0:
        q, s, wdq = f16(wf), None, f16(wf)
    else:
        q, s = hxo.q8_quantize(wf) if fmt == 1 else hxo.q4_quantize(wf)
        wdq = hxo.q8_dequant(q, s) if fmt == 1 else hxo.q4_dequant(q, s)
    dA, dW = hip.DeviceArray.from_numpy(A), hip.DeviceArray.from_numpy(q)
    dS = hip.DeviceArray.from_numpy(s) if s is not None else None
    out = hip.DeviceArray((S, M, N), np.float32)
    args = (dA.ptr, K, M, fmt, dW.ptr, dS.ptr if dS else None, None, N, K, S, hip.EPI_PARTIAL_F32, out.ptr, N, M * N,
            None, 0, None)
    if tile:
        hip.check(hip.lib().hxa_gemm_tile(*args, tile[0], tile[1], tile[2], None), "gemm_tile")
    else:
        hip.check(hip.lib().hxa_gemm(*args, None, 0, 0, None), "gemm")
    hip.sync()
    got = out.numpy()
    W16 = np.asarray(wdq).view(np.float16)
    for z in range(S):
        sl = slice(z * K // S, (z + 1) * K // S)
        ref = hxo.gemm(A[:, sl], wdq[:, sl]).astype(np.float64)
        absdot = hxo.gemm(np.abs(A[:, sl]), np.abs(W16[:, sl])).astype(np.float64)
        tol = absdot * 4.0 * np.sqrt(K / S) * 2.0 ** -24 + np.abs(ref) * 2.0 ** -24
        err = np.abs(got[z].astype(np.float64) - ref)
        assert np.all(err <= tol), f"slice {z}: max excess {np.max(err - tol):.3e}"


@pytest.mark.parametrize("N,K", [(2048, 8192), (2560, 10240), (6144, 2048), (3072, 12288)])
@pytest.mark.parametrize("fmt", [0, 1, 2])
def test_linear_config1_shapes(N, K, fmt):
    """hxa_linear at M = 1536 on the long-K shapes it splits (8192 x 2048, 10240 x 2560, 12288 x 3072) and one it
    runs as one launch (2048 x 6144): against the oracle's dequantised-fp16 GEMM with the one-launch GEMM's
    tolerance (one ulp + accumulation bound, >= 98% bit-identical), and against hxa_gemm's one-launch output (>= 98%
    bit-identical; the outputs that differ are fp32 summation-order differences, inside the same bound, so near-zero
    sums from cancellation may differ by many of their own small ulps)."""
    hip = _hip()
    L = hip.lib()
    M = 1536
    nsplit = L.hxa_linear_split_k(M, N, K, fmt)
    say(f"linear fmt={fmt} M={M} N={N} K={K} split={nsplit}")
    if K >= 4 * N:
        assert nsplit > 1
    rng = np.random.default_rng(N + K + 10 * fmt)
    A = f16(rng.standard_normal((M, K)))
    wf = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    if fmt == 0:
        q, s, wdq = f16(wf), None, f16(wf)
    else:
        q, s = hxo.q8_quantize(wf) if fmt == 1 else hxo.q4_quantize(wf)
        wdq = hxo.q8_dequant(q, s) if fmt == 1 else hxo.q4_dequant(q, s)
    dA, dW = hip.DeviceArray.from_numpy(A), hip.DeviceArray.from_numpy(q)
    dS = hip.DeviceArray.from_numpy(s) if s is not None else None
    wsb = L.hxa_linear_ws_bytes(M, N, K, fmt)
    assert wsb == (nsplit * M * N * 4 if nsplit > 1 else 0)
    ws = hip.DeviceArray((max(wsb, 16),), np.uint8)
    out = hip.DeviceArray((M, N), np.float16)
    one = hip.DeviceArray((M, N), np.float16)
    sp = dS.ptr if dS else None
    hip.check(L.hxa_linear(dA.ptr, K, M, fmt, dW.ptr, sp, None, N, K, out.ptr, N, ws.ptr, wsb, None), "linear")
    hip.check(L.hxa_gemm(dA.ptr, K, M, fmt, dW.ptr, sp, None, N, K, 1, hip.EPI_STORE, one.ptr, N, 0, None, 0, None,
                         None, 0, 0, None), "gemm")
    hip.sync()
    got, g1 = out.numpy(), one.numpy()
    assert_gemm_close(got, hxo.gemm(A, wdq), A, np.asarray(wdq).view(np.float16))
    same = np.mean(got.view(np.uint16) == g1.view(np.uint16))
    assert same >= 0.98, same


@pytest.mark.parametrize("fmt,asym", [(1, False), (2, True)])
def test_linear_split_ragged_padded_and_fallback(fmt, asym):
    """hxa_linear's split form with ragged rows (M = 1000), a padded output (ldo = N + 64, padding untouched) and int4
    with mins (q4a): against the oracle's dequantised-fp16 GEMM; with a workspace one byte short it runs the one-launch
    form, bit for bit hxa_gemm's output."""
    hip = _hip()
    L = hip.lib()
    M, N, K, ldo = 1000, 2048, 8192, 2048 + 64
    nsplit = L.hxa_linear_split_k(M, N, K, fmt)
    say(f"linear fmt={fmt} asym={asym} M={M} N={N} K={K} ldo={ldo} split={nsplit}")
    assert nsplit > 1
    rng = np.random.default_rng(300 + fmt)
    A = f16(rng.standard_normal((M, K)))
    if asym:
        q, s, z = _q4a_weights(rng, N, K)
        wdq = hxo.q4_dequant(q, s, z)
    else:
        q, s = hxo.q8_quantize((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
        z, wdq = None, hxo.q8_dequant(q, s)
    dA, dW, dS = hip.DeviceArray.from_numpy(A), hip.DeviceArray.from_numpy(q), hip.DeviceArray.from_numpy(s)
    dZ = hip.DeviceArray.from_numpy(z) if z is not None else None
    zp = dZ.ptr if dZ else None
    wsb = L.hxa_linear_ws_bytes(M, N, K, fmt)
    ws = hip.DeviceArray((wsb,), np.uint8)
    pad = np.full((M, ldo), np.float16(3.0))
    outs = []
    for nbytes in (wsb, wsb - 1):
        out = hip.DeviceArray.from_numpy(pad)
        hip.check(L.hxa_linear(dA.ptr, K, M, fmt, dW.ptr, dS.ptr, zp, N, K, out.ptr, ldo, ws.ptr, nbytes, None),
                  "linear")
        outs.append(out)
    one = hip.DeviceArray((M, N), np.float16)
    hip.check(L.hxa_gemm(dA.ptr, K, M, fmt, dW.ptr, dS.ptr, zp, N, K, 1, hip.EPI_STORE, one.ptr, N, 0, None, 0, None,
                         None, 0, 0, None), "gemm")
    hip.sync()
    split, short = outs[0].numpy(), outs[1].numpy()
    assert np.all(split[:, N:] == np.float16(3.0)) and np.all(short[:, N:] == np.float16(3.0))
    assert_gemm_close(split[:, :N], hxo.gemm(A, wdq), A, np.asarray(wdq).view(np.float16))
    assert np.array_equal(short[:, :N].view(np.uint16), one.numpy().view(np.uint16))
    assert L.hxa_linear(dA.ptr, K, M, fmt, dW.ptr, dS.ptr, zp, N, K, one.ptr, N - 8, ws.ptr, wsb, None) != 0
