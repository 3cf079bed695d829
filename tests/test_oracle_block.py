"""Block-level pinning of the oracle: the composed Anima and MOSS blocks against float64 numpy restatements of the
reference's own torch blocks (moss/moss_ref.py:56-67 `block`; the Anima block's site order from
hexagon/mega/blk.c:149-176 and export_block.py's FullBlock call), and structural invariants (zero gates leave x
unchanged, stop-after-stage semantics of meta[M_STOP], masked joint-attention keys have no influence)."""
import numpy as np
import pytest

from oracle import hxo


def f16(a):
    return np.asarray(a).astype(np.float16)


def _ln(x):
    mu = x.mean(-1, keepdims=True)
    return (x - mu) / np.sqrt((x * x).mean(-1, keepdims=True) - mu * mu + 1e-6)


def _rms(x, w):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6) * w


def _rope(x, cos, sin):
    # moss_ref.py:37-39 rotate: x*cos + cat(-b, a)*sin over halves of 128, cos/sin duplicated to 128
    a, b = x[..., :64], x[..., 64:]
    c, s = cos[:, None, :], sin[:, None, :]
    return np.concatenate([a * c - b * s, b * c + a * s], -1)


def _attn(q, k, v, nvalid=None):
    T, D = q.shape
    H = D // 128
    nv = k.shape[0] if nvalid is None else nvalid
    qh, kh, vh = q.reshape(T, H, 128), k[:nv].reshape(nv, H, 128), v[:nv].reshape(nv, H, 128)
    S = np.einsum("thd,shd->hts", qh, kh)
    P = np.exp(S - S.max(-1, keepdims=True))
    P /= P.sum(-1, keepdims=True)
    return np.einsum("hts,shd->thd", P, vh).reshape(T, D)


def _gelu_tanh(x):
    return 0.5 * x * (1 + np.tanh(np.sqrt(2 / np.pi) * (x + 0.044715 * x ** 3)))


def anima_block_f64(x, ctx, mod9, cos, sin, w, H):
    """float64 restatement of the Anima block (no fp16 storage rounding)."""
    d = lambda k: w[k].astype(np.float64)
    g = w["gain"].astype(np.float64).reshape(4, 128)
    T, D = x.shape
    m = mod9.astype(np.float64).reshape(9, D)
    x = x.astype(np.float64).copy()
    ctxd = ctx.astype(np.float64)
    # site 0
    h = _ln(x) * (1 + m[1]) + m[0]
    q = _rope(_rms((h @ d("wq").T).reshape(T, H, 128), g[0]), cos, sin).reshape(T, D)
    k = _rope(_rms((h @ d("wk").T).reshape(T, H, 128), g[1]), cos, sin).reshape(T, D)
    v = h @ d("wv").T
    x = x + m[2] * (_attn(q, k, v) @ d("wo").T)
    # site 1
    h = _ln(x) * (1 + m[4]) + m[3]
    q = _rms((h @ d("wcq").T).reshape(T, H, 128), g[2]).reshape(T, D)
    ck = _rms((ctxd @ d("wck").T).reshape(len(ctxd), H, 128), g[3]).reshape(len(ctxd), D)
    cv = ctxd @ d("wcv").T
    x = x + m[5] * (_attn(q, ck, cv) @ d("wco").T)
    # site 2
    h = _ln(x) * (1 + m[7]) + m[6]
    x = x + m[8] * (_gelu_tanh(h @ d("w1").T) @ d("w2").T)
    return x


def make_anima(T=128, D=256, H=2, C=64, DC=128, F=512, seed=0, gh=8):
    rng = np.random.default_rng(seed)
    w = {}
    for k, (n, kk) in {"wq": (D, D), "wk": (D, D), "wv": (D, D), "wo": (D, D), "wcq": (D, D), "wck": (D, DC),
                       "wcv": (D, DC), "wco": (D, D), "w1": (F, D), "w2": (D, F)}.items():
        w[k] = f16(rng.standard_normal((n, kk)) * 0.02 * np.sqrt(2048 / kk))
    w["gain"] = np.concatenate([rng.uniform(0.5, 1.5, 128) / np.sqrt(128), rng.uniform(0.5, 1.5, 128),
                                rng.uniform(0.5, 1.5, 128) / np.sqrt(128), rng.uniform(0.5, 1.5, 128)]).astype(np.float32)
    x = rng.standard_normal((T, D)).astype(np.float32)
    ctx = f16(rng.standard_normal((C, DC)))
    mod9 = (rng.standard_normal((9, D)) * 0.3).astype(np.float32)
    cos, sin = hxo.rope_anima(gh, T // gh)
    return x, ctx, mod9, cos, sin, w


def test_anima_block_vs_float64_restatement():
    x, ctx, mod9, cos, sin, w = make_anima()
    ref = anima_block_f64(x, ctx, mod9, cos, sin, w, H=2)
    for mode in (0, 1):
        out, buf, n = hxo.anima_block(x, ctx, mod9, cos, sin, w, H=2, F=512, gelu=1, attn_mode=mode)
        assert n == 13
        dl = ref - x
        rel = np.linalg.norm(out - ref) / np.linalg.norm(dl)
        cos_d = np.dot((out - x).ravel(), dl.ravel()) / np.linalg.norm(out - x) / np.linalg.norm(dl)
        assert rel < 5e-3, rel
        assert cos_d > 0.99998, cos_d


def test_anima_zero_gates_and_stop_semantics():
    x, ctx, mod9, cos, sin, w = make_anima(seed=1)
    m = mod9.copy()
    m[[2, 5, 8]] = 0.0
    out, _, n = hxo.anima_block(x, ctx, m, cos, sin, w, H=2, F=512)
    assert n == 13 and np.array_equal(out, x)
    # stop after stage 5 (site 0 finished) == a block whose sites 1, 2 have zero gates
    out5, buf5, n5 = hxo.anima_block(x, ctx, mod9, cos, sin, w, H=2, F=512, stop=5)
    m2 = mod9.copy()
    m2[[5, 8]] = 0.0
    full, buf, _ = hxo.anima_block(x, ctx, m2, cos, sin, w, H=2, F=512)
    assert n5 == 5 and np.array_equal(out5, full)
    # stop after stage 1: only h written, x untouched
    out1, buf1, n1 = hxo.anima_block(x, ctx, mod9, cos, sin, w, H=2, F=512, stop=1)
    assert n1 == 1 and np.array_equal(out1, x)
    assert np.array_equal(buf1["h"], hxo.lnmod(x, mod9[0], mod9[1]))
    assert not buf1["q"].any()
    # stop after stage 2: q is the raw projection, stage 3 applies RMS + RoPE in place
    _, b2, _ = hxo.anima_block(x, ctx, mod9, cos, sin, w, H=2, F=512, stop=2)
    _, b3, _ = hxo.anima_block(x, ctx, mod9, cos, sin, w, H=2, F=512, stop=3)
    assert np.array_equal(b3["q"], hxo.rmsrope(b2["q"], w["gain"][:128], cos, sin))


def test_anima_gelu_modes_differ_only_in_mlp():
    x, ctx, mod9, cos, sin, w = make_anima(seed=2)
    a, ba, _ = hxo.anima_block(x, ctx, mod9, cos, sin, w, H=2, F=512, gelu=0)
    b, bb, _ = hxo.anima_block(x, ctx, mod9, cos, sin, w, H=2, F=512, gelu=1)
    assert np.array_equal(ba["o"], bb["o"])  # sites 0/1 identical
    assert not np.array_equal(ba["mid"], bb["mid"])
    assert np.linalg.norm(a - b) / np.linalg.norm(b - x) < 5e-2  # erf vs tanh GELU are close


def moss_block_f64(x, mod6, cos, sin, w, nvalid):
    """float64 restatement of moss_ref.py:56-67 block (no LoRA), attention over the valid tokens only."""
    d = lambda k: w[k].astype(np.float64)
    T, D = x.shape
    H = D // 128
    sa, ca, ga, sf, cf, gf = mod6.astype(np.float64).reshape(6, D)
    x = x.astype(np.float64).copy()
    y = _rms(x, w["n1"]) * (1 + ca) + sa
    q = _rope(_rms((y @ d("wq").T).reshape(T, H, 128), w["gq"]), cos, sin).reshape(T, D)
    k = _rope(_rms((y @ d("wk").T).reshape(T, H, 128), w["gk"]), cos, sin).reshape(T, D)
    v = y @ d("wv").T
    x = x + (_attn(q, k, v, nvalid) @ d("wo").T) * ga
    y = _rms(x, w["n2"]) * (1 + cf) + sf
    up, gt = y @ d("wup").T, y @ d("wgate").T
    mid = (4.0 * np.tanh(gt / 4.0) / (1 + np.exp(-gt))) * (25.0 * np.tanh(up / 25.0))
    return x + (mid @ d("wdown").T) * gf


def make_moss(T=160, nvalid=150, D=256, F=512, seed=0):
    rng = np.random.default_rng(seed)
    w = {k: f16(rng.standard_normal((n, kk)) * 0.02 * np.sqrt(3072 / kk)) for k, (n, kk) in
         {"wq": (D, D), "wk": (D, D), "wv": (D, D), "wo": (D, D), "wup": (F, D), "wgate": (F, D), "wdown": (D, F)}.items()}
    w["gq"] = (rng.uniform(0.5, 1.5, 128) / np.sqrt(128)).astype(np.float32)
    w["gk"] = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    w["n1"] = rng.uniform(0.5, 1.5, D).astype(np.float32)
    w["n2"] = rng.uniform(0.5, 1.5, D).astype(np.float32)
    x = (rng.standard_normal((T, D)) * 4).astype(np.float32)
    mod6 = (rng.standard_normal((6, D)) * 0.3).astype(np.float32)
    bands = (1.0 / 10000.0 ** (np.arange(16) / 16)).astype(np.float32)
    cos, sin = hxo.rope_moss(10, 12, 30, bands)  # 120 image + 30 text = 150 valid tokens
    cos = np.concatenate([cos, np.ones((T - len(cos), 64), np.float32)])
    sin = np.concatenate([sin, np.zeros((T - len(sin), 64), np.float32)])
    return x, mod6, cos, sin, w


def test_moss_block_vs_float64_restatement():
    x, mod6, cos, sin, w = make_moss()
    nv = 150
    ref = moss_block_f64(x, mod6, cos, sin, w, nv)
    out, buf, n = hxo.moss_block(x, mod6, cos, sin, w, H=2, F=512, nvalid=nv)
    assert n == 8
    dl = (ref - x)[:nv]
    rel = np.linalg.norm((out - ref)[:nv]) / np.linalg.norm(dl)
    assert rel < 6e-3, rel
    # padded rows never influence valid rows
    x2 = x.copy()
    x2[nv:] = 123.0
    out2, _, _ = hxo.moss_block(x2, mod6, cos, sin, w, H=2, F=512, nvalid=nv)
    assert np.array_equal(out2[:nv], out[:nv])


@pytest.mark.parametrize("stop", [1, 4, 5, 8])
def test_moss_stop(stop):
    x, mod6, cos, sin, w = make_moss(seed=3)
    out, buf, n = hxo.moss_block(x, mod6, cos, sin, w, H=2, F=512, nvalid=150, stop=stop)
    assert n == stop
    if stop < 5:
        assert np.array_equal(out, x)
    else:
        assert not np.array_equal(out, x)


def make_moss_lora(T=160, nvalid=150, D=256, F=512, seed=5, scale=0.75, bzero=False):
    """A MOSS block with the rapid-moss LoRA in the reference's torch form (moss_ref.py:44-50 `lin`: per projection
    A [r][in], B [out][r], scale s) and in the packed form the oracle / GPU take (moss/export_moss.py:34-47 `mat`:
    the rows of f16(s B) appended after K, A_qkv = cat(A_q, A_k, A_v))."""
    x, mod6, cos, sin, w = make_moss(T, nvalid, D, F, seed)
    rng = np.random.default_rng(seed + 100)
    R = hxo.LORA_R
    ins = {"q": D, "k": D, "v": D, "o": D, "up": D, "gate": D, "down": F}
    A = {n: f16(rng.standard_normal((R, k)) * 0.05) for n, k in ins.items()}
    A["gate"] = A["up"]  # one LoRA on the fused up_gate projection (moss_ref.py:64)
    B = {n: f16(rng.standard_normal((w["w" + n].shape[0], R)) * (0.0 if bzero else 0.05)) for n in ins}
    Bs = {n: f16(scale * B[n].astype(np.float32)) for n in ins}  # s B rounded to the pack's storage
    wl = dict(w)
    for n in ins:
        wl["w" + n] = np.ascontiguousarray(np.concatenate([w["w" + n], Bs[n]], 1))
    wl["aqkv"] = np.ascontiguousarray(np.concatenate([A["q"], A["k"], A["v"]], 0))
    wl["ao"], wl["aug"], wl["adn"] = A["o"], A["up"], A["down"]
    return x, mod6, cos, sin, w, wl, A, Bs


def moss_block_lora_f64(x, mod6, cos, sin, w, A, Bs, nvalid):
    """float64 restatement of moss_ref.py:56-67 `block` with `lin(x, W, lora=(A, B, s))` = x W^T + s (x A^T) B^T."""
    d = lambda a: np.asarray(a).astype(np.float64)
    lin = lambda y, n: y @ d(w["w" + n]).T + (y @ d(A[n]).T) @ d(Bs[n]).T
    T, D = x.shape
    H = D // 128
    sa, ca, ga, sf, cf, gf = mod6.astype(np.float64).reshape(6, D)
    x = x.astype(np.float64).copy()
    y = _rms(x, w["n1"]) * (1 + ca) + sa
    q = _rope(_rms(lin(y, "q").reshape(T, H, 128), w["gq"]), cos, sin).reshape(T, D)
    k = _rope(_rms(lin(y, "k").reshape(T, H, 128), w["gk"]), cos, sin).reshape(T, D)
    v = lin(y, "v")
    x = x + lin(_attn(q, k, v, nvalid), "o") * ga
    y = _rms(x, w["n2"]) * (1 + cf) + sf
    up, gt = lin(y, "up"), lin(y, "gate")
    mid = (4.0 * np.tanh(gt / 4.0) / (1 + np.exp(-gt))) * (25.0 * np.tanh(up / 25.0))
    return x + lin(mid, "down") * gf


def test_moss_lora_block_vs_float64_restatement():
    """The oracle's [x | L] . [W ; s B] form (moss/hexagon/mega/blk.c:238-259) against the torch reference's
    x W^T + s (x A^T) B^T: the q / k / v parts of L feed their own projections, the down projection's LoRA rides on
    its second K half. The LoRA term is large enough here that a dropped or misrouted part fails the bound."""
    x, mod6, cos, sin, w, wl, A, Bs = make_moss_lora()
    nv = 150
    ref = moss_block_lora_f64(x, mod6, cos, sin, w, A, Bs, nv)
    out, buf, n = hxo.moss_block(x, mod6, cos, sin, wl, H=2, F=512, nvalid=nv)
    assert n == 8
    dl = (ref - x)[:nv]
    rel = np.linalg.norm((out - ref)[:nv]) / np.linalg.norm(dl)
    assert rel < 6e-3, rel
    nolora = moss_block_f64(x, mod6, cos, sin, w, nv)
    assert np.linalg.norm((nolora - ref)[:nv]) / np.linalg.norm(dl) > 20 * rel  # the LoRA term is not negligible


def test_moss_lora_with_zero_b_is_the_plain_block():
    """B = 0: [x | L] . [W ; 0] accumulates exact zeros after the W part, so the block is bit-identical to the
    block without LoRA."""
    x, mod6, cos, sin, w, wl, A, Bs = make_moss_lora(bzero=True)
    out, _, _ = hxo.moss_block(x, mod6, cos, sin, wl, H=2, F=512, nvalid=150)
    plain, _, _ = hxo.moss_block(x, mod6, cos, sin, w, H=2, F=512, nvalid=150)
    assert np.array_equal(out, plain)


def test_glue_oracle_bn_unpatchify_and_rms_vec():
    """The rapid-moss output step (mossrun.cpp:339-343) restated by loops on a tiny case: zo[c/4][2h + (c/2)%2]
    [2w + c%2] = x0[c][h][w] sqrt(var[c] + 1e-4) + mean[c]; and the t-embedding RMSNorm (animad.cpp:115-123)
    against float64 with a one-hot input (the norm of a one-hot vector of value a is sqrt(n) sign(a) w)."""
    from tests._helpers import bn_unpatchify, rms_vec
    rng = np.random.default_rng(3)
    Cc, H, W = 2, 4, 6
    x0 = rng.standard_normal((H // 2 * W // 2, 4 * Cc)).astype(np.float32)  # token rows [T][128-channel]
    mean, var = rng.standard_normal(4 * Cc).astype(np.float32), rng.uniform(0.5, 2, 4 * Cc).astype(np.float32)
    want = np.zeros((Cc, H, W), np.float64)
    for c in range(4 * Cc):
        for h in range(H // 2):
            for w in range(W // 2):
                want[c // 4, 2 * h + (c // 2) % 2, 2 * w + c % 2] = x0[h * (W // 2) + w, c] * np.sqrt(var[c] + 1e-4) + mean[c]
    assert np.allclose(bn_unpatchify(x0, mean, var, Cc, H, W), want, rtol=1e-6, atol=1e-6)
    n = 64
    wv = f16(rng.uniform(0.5, 1.5, n))
    e = np.zeros(n, np.float32)
    e[5] = -3.0
    y = rms_vec(e, wv.view(np.uint16))
    assert abs(y[5] - (-np.sqrt(n) * float(wv[5]))) < 1e-4 and np.count_nonzero(y) == 1
