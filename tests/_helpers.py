"""Shared helpers of the parity tests: comparison metrics (the reference's own: hexagon/mega/cmp_block.py:5-6
rel err on the block delta + cosine; moss/cmp_blk.py:9 per-stage rel err), GPU-pack <-> oracle-weight conversion
and an oracle-composed DiT step (the caller-side glue of phone/animad.cpp:424-492 around the oracle blocks)."""
import numpy as np

from oracle import hxo
from hexanima_amd import hip


def f16(a):
    return np.asarray(a).astype(np.float16)


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / (np.linalg.norm(b) + 1e-30))


def delta_metrics(out, ref, x0):
    """cmp_block.py:5-6: rel err on the block delta and cosine of the deltas."""
    out, ref, x0 = (np.asarray(v, np.float64) for v in (out, ref, x0))
    dl = ref - x0
    do = out - x0
    r = float(np.linalg.norm(out - ref) / np.linalg.norm(dl))
    c = float(do.ravel() @ dl.ravel() / (np.linalg.norm(do) * np.linalg.norm(dl)))
    return r, c


def ulp_diff(a16, b16):
    """max distance in fp16 ulps between two fp16 arrays (same sign assumed)."""
    a = np.asarray(a16).view(np.uint16).astype(np.int32)
    b = np.asarray(b16).view(np.uint16).astype(np.int32)
    sa = np.where(a & 0x8000, -(a & 0x7FFF), a)
    sb = np.where(b & 0x8000, -(b & 0x7FFF), b)
    return np.abs(sa - sb)


def unpack_weights(pack: np.ndarray, kind: int, D: int, F: int, DC: int, fmt_attn: int, fmt_mlp: int, layout):
    """GPU pack image (k-tiled matrices) -> dict of fp16 (uint16) W[N][K] matrices (dequantised) and the fp32
    vector section."""
    total, offs, voff = layout
    shapes = hip.pack_shapes(kind, D, F, DC)
    fmts = hip.pack_fmts(kind, fmt_attn, fmt_mlp)
    mats = []
    for i, ((N, K), (wo, so)) in enumerate(zip(shapes, offs)):
        fmt = fmts[i]
        if fmt == 0:
            mats.append(hip.unktile(pack[wo:wo + N * K * 2], N, K).view(np.uint16).reshape(N, K).copy())
        else:
            s = pack[so:so + (K // 32) * N * 2].view(np.uint16).reshape(K // 32, N).copy()
            if fmt == 1:
                q = hip.unktile(pack[wo:wo + N * K], N, K).view(np.int8).reshape(N, K).copy()
                mats.append(hxo.q8_dequant(q, s))
            else:
                q = hip.unktile(pack[wo:wo + N * K // 2], N, K).reshape(N, K // 2).copy()
                mats.append(hxo.q4_dequant(q, s))
    if kind == 0:
        qkv, wo_, wcq, ckv, wco, w1, w2 = mats
        vec = pack[voff:voff + 4 * 512].view(np.float32).copy()
        return {"wq": qkv[:D], "wk": qkv[D:2 * D], "wv": qkv[2 * D:], "wo": wo_, "wcq": wcq, "wck": ckv[:D],
                "wcv": ckv[D:], "wco": wco, "w1": w1, "w2": w2, "gain": vec}
    qkv, wo_, ug, dn = mats[:4]
    vec = pack[voff:voff + 4 * (256 + 2 * D)].view(np.float32).copy()
    K1 = ug.shape[1]
    ugr = ug.reshape(F // 32, 2, 32, K1)
    out = {"wo": wo_, "wup": np.ascontiguousarray(ugr[:, 0].reshape(F, K1)),
           "wgate": np.ascontiguousarray(ugr[:, 1].reshape(F, K1)), "wdown": dn, "gq": vec[:128], "gk": vec[128:256],
           "n1": vec[256:256 + D], "n2": vec[256 + D:]}
    if kind == 1:
        out.update({"wq": qkv[:D], "wk": qkv[D:2 * D], "wv": qkv[2 * D:]})
    else:  # block-diagonal LoRA columns of the fused qkv -> [W | s B] per projection (the oracle's form)
        R = hip.LORA_R
        for p, n in enumerate(("wq", "wk", "wv")):
            rows = qkv[p * D:(p + 1) * D]
            out[n] = np.ascontiguousarray(np.concatenate([rows[:, :D], rows[:, D + p * R:D + (p + 1) * R]], 1))
        out.update({"aqkv": mats[4], "ao": mats[5], "aug": mats[6], "adn": mats[7]})
    return out


def silu(v):
    v = np.asarray(v, np.float64)
    return (v / (1.0 + np.exp(-v))).astype(np.float32)


def oracle_anima_velocity(lat, ctx16, sigma, blocks, modws, glue, *, D, H, F, C4, temb, gelu=1, attn_mode=0):
    """v(x, sigma) of the Anima-structure DiT, image by image, from the oracle primitives.
    glue = (Wemb [D][C4], L1 [D][temb], Lf [2D][D], Wfin [C4][D]) fp16; modws[k] [6D][D] fp16."""
    Wemb, L1, Lf, Wfin = glue
    B, Cc, Hl, Wl = lat.shape
    s = hxo.sinusoid(sigma, temb)
    c = hxo.linear_f32(s[None, :], L1)
    sc = silu(c)
    mods = []
    for mw in modws:
        m6 = hxo.linear_f32(sc, mw)[0].reshape(6, D)
        mods.append(np.concatenate([m6[:3], np.zeros((2, D), np.float32), np.ones((1, D), np.float32), m6[3:]]))
    fm = hxo.linear_f32(sc, Lf)[0]
    cos, sin = hxo.rope_anima(Hl // 2, Wl // 2)
    out = np.zeros_like(lat)
    for b in range(B):
        x = hxo.linear_f32(hxo.patchify(lat[b]), Wemb)
        for w, m9 in zip(blocks, mods):
            x, _, _ = hxo.anima_block(x, ctx16[b], m9, cos, sin, w, H=H, F=F, gelu=gelu, attn_mode=attn_mode)
        xn = hxo.final_norm(x, fm[:D], fm[D:])
        out[b] = hxo.unpatchify(hxo.linear_f32(xn, Wfin), Cc, Hl, Wl)
    return out


def oracle_moss_velocity(lat, txt16, sigma, blocks, modw, glue, *, D, H, F, C4, temb, ntxt, Ttot, attn_mode=0):
    """v(x, sigma) of the MOSS-class DiT (moss_ref.py:56-67 blocks with one shared modulation, joint image + text
    attention over nvalid = image + text tokens, padded to Ttot), image by image, from the oracle primitives.
    glue = (Wemb [D][C4], L1 [D][temb], Lf [2D][D], Wfin [C4][D], Wtxt [D][ntxt_in]) fp16; modw [6D][D] fp16.
    The text rows are f16(text . Wtxt^T) (the projection written into zeroed rows, moss blk.c MODE 2)."""
    Wemb, L1, Lf, Wfin, Wtxt = glue
    B, Cc, Hl, Wl = lat.shape
    s = hxo.sinusoid(sigma, temb)
    sc = silu(hxo.linear_f32(s[None, :], L1))
    mod6 = hxo.linear_f32(sc, modw)[0].reshape(6, D)
    fm = hxo.linear_f32(sc, Lf)[0]
    bands = (1.0 / 10000.0 ** (np.arange(16) / 16.0)).astype(np.float32)
    c, sn = hxo.rope_moss(Hl // 2, Wl // 2, ntxt, bands)
    cos = np.ones((Ttot, 64), np.float32)
    sin = np.zeros((Ttot, 64), np.float32)
    cos[:c.shape[0]], sin[:c.shape[0]] = c, sn
    timg = (Hl // 2) * (Wl // 2)
    out = np.zeros_like(lat)
    for b in range(B):
        x = np.zeros((Ttot, D), np.float32)
        x[:timg] = hxo.linear_f32(hxo.patchify(lat[b]), Wemb)
        x[timg:timg + ntxt] = f16(hxo.gemm(txt16[b], Wtxt)).astype(np.float32)
        for w in blocks:
            x, _, _ = hxo.moss_block(x, mod6, cos, sin, w, H=H, F=F, nvalid=timg + ntxt, attn_mode=attn_mode)
        xn = hxo.final_norm(x[:timg], fm[:D], fm[D:])
        out[b] = hxo.unpatchify(hxo.linear_f32(xn, Wfin), Cc, Hl, Wl)
    return out


def gemm_bound(A16, W16):
    """Per-element bound on |f16(fp32-accumulated A.W^T) - f16(exact)|: one fp16 ulp of the result plus the fp32
    accumulation-order error 4 sqrt(K) 2^-24 sum_k |a_k w_k| (probabilistic form of the gamma_K bound)."""
    K = A16.shape[1]
    absdot = hxo.gemm(np.abs(np.asarray(A16, np.float16)), np.abs(np.asarray(W16, np.float16))).astype(np.float64)
    return absdot * 4.0 * np.sqrt(K) * 2.0 ** -24


def assert_gemm_close(got16, ref32, A16, W16, ident=0.98):
    """GEMM parity: |got - f16(ref)| <= ulp(|ref|) + accumulation bound, and >= ident of the outputs bit-identical."""
    g = np.asarray(got16, np.float16).astype(np.float64)
    r16 = np.asarray(ref32, np.float32).astype(np.float16)
    r = r16.astype(np.float64)
    ulp = np.spacing(np.maximum(np.abs(r), 2.0 ** -14).astype(np.float16)).astype(np.float64)
    tol = ulp + gemm_bound(A16, W16)
    err = np.abs(g - r)
    assert np.all(err <= tol), f"max excess {np.max(err - tol):.3e}"
    same = np.mean(np.asarray(got16, np.float16).view(np.uint16) == r16.view(np.uint16))
    assert same >= ident, f"only {same:.4f} bit-identical"


def oracle_anima_modulation(modw16, emb, lora):
    """megarun.cpp:156-171: s = silu(emb); per site: h1 = A_site s, mod rows 3 site .. 3 site + 2 = lora + B_site h1
    (fp32 activations, fp16 weights). modw16: the W_MODW section of a blkNN.bin as uint16, per site A [256][2048]
    then B [6144][256] (export_all.py:59-61). Returns [9][2048] fp32."""
    out = []
    s = silu(np.asarray(emb, np.float32))[None, :]
    step = 256 * 2048 + 6144 * 256
    for site in range(3):
        a = modw16[site * step:site * step + 256 * 2048].reshape(256, 2048)
        b = modw16[site * step + 256 * 2048:(site + 1) * step].reshape(6144, 256)
        h1 = hxo.linear_f32(s, a)
        out.append(np.asarray(lora, np.float32) + hxo.linear_f32(h1, b)[0])
    return np.concatenate(out).reshape(9, 2048).astype(np.float32)


def rms_vec(x, w16, eps=1e-6):
    """animad.cpp:115-123 rms_rows on one vector: x * 1 / sqrt(sum(x^2) / n + eps) (sum in double) * w (fp16)."""
    x = np.asarray(x, np.float32)
    s = float(np.sum(x.astype(np.float64) ** 2))
    k = np.float32(1.0) / np.sqrt(np.float32(s / x.size) + np.float32(eps))
    return (x * k * np.asarray(w16).view(np.float16).astype(np.float32)).astype(np.float32)


def oracle_anima_ref_velocity(lat, ctx16, sigma, blocks, modws, glue, *, D, H, F, C4, gelu=1, attn_mode=0):
    """v(x, sigma) of the Anima DiT with the reference's own glue, image by image:
    t-embedding (animad.cpp:424-431): tp = sinusoid_D(t), emb = RMSNorm(tp) * t_norm, lora = L2 silu(L1 tp);
    per block and site (megarun.cpp:159-167): mod = lora + B (A silu(emb)); final (animad.cpp:475-492): (shift, scale) =
    F2 (F1 silu(emb)) + lora[:2D], LN(x) (1 + scale) + shift, linear, unpatchify.
    glue = (Wemb [D][C4], L1 [D][D], L2 [3D][D], F1 [256][D], F2 [2D][256], Wfin [C4][D], t_norm [D]) fp16;
    modws[k] = (A [3*256][D], B [3][3D][256]) fp16."""
    Wemb, L1, L2, F1, F2, Wfin, tnorm = glue
    B_, Cc, Hl, Wl = lat.shape
    tp = hxo.sinusoid(sigma, D)
    emb = rms_vec(tp, tnorm)
    lora = hxo.linear_f32(silu(hxo.linear_f32(tp[None, :], L1)), L2)[0]
    se = silu(emb)[None, :]
    mods = []
    for A, Bm in modws:
        rows = []
        for site in range(3):
            h1 = hxo.linear_f32(se, A[site * 256:(site + 1) * 256])
            rows.append(lora + hxo.linear_f32(h1, np.ascontiguousarray(Bm[site]))[0])
        mods.append(np.concatenate(rows).reshape(9, D).astype(np.float32))
    fm = hxo.linear_f32(hxo.linear_f32(se, F1), F2)[0] + lora[:2 * D]
    cos, sin = hxo.rope_anima(Hl // 2, Wl // 2)
    out = np.zeros_like(lat)
    for b in range(B_):
        x = hxo.linear_f32(hxo.patchify(lat[b]), Wemb)
        for w, m9 in zip(blocks, mods):
            x, _, _ = hxo.anima_block(x, ctx16[b], m9, cos, sin, w, H=H, F=F, gelu=gelu, attn_mode=attn_mode)
        xn = hxo.final_norm(x, fm[:D], fm[D:])
        out[b] = hxo.unpatchify(hxo.linear_f32(xn, Wfin), Cc, Hl, Wl)
    return out


def lin(x, W):
    """x W^T: fp16 weights (uint16 bits) through the oracle's fp32 linear; fp32 weights (the MOSS glue's fp32
    tensors, moss/export_glue.py:7-12) in float64, rounded once to fp32."""
    if W.dtype == np.uint16:
        return hxo.linear_f32(x, W)
    return (np.asarray(x, np.float64) @ np.asarray(W, np.float64).T).astype(np.float32)


def moss_ref_sections(glue16, vec32, D, C4, tin):
    """The MOSS reference form's exported glue sections (hxa_dit_export 2 nb: fp16 head_mod [2D][D] | text_proj
    [D][tin]; 2 nb + 1: fp32 vectors then video_embed [D][C4] | t0 [D][256] | t2 [D][D] | final_linear [C4][D]) ->
    (glue, vec) as oracle_moss_rapid_step takes them."""
    Wh, Wt = split_flat(glue16, [(2 * D, D), (D, tin)])
    v = split_flat(vec32, [(D,), (D,), (D,), (6 * D,), (2 * D,), (D,), (C4, C4), (C4,), (C4,), (D, C4), (D, 256),
                           (D, D), (C4, D)])
    return (v[9], v[10], v[11], Wh, v[12], Wt), v[:9]


def split_flat(buf, shapes):
    out, o = [], 0
    for sh in shapes:
        n = int(np.prod(sh))
        out.append(buf[o:o + n].reshape(sh))
        o += n
    assert o == buf.size
    return out


def oracle_moss_rapid_step(z, x0, txt16, code, blocks, modw, glue, vec, *, D, H, F, C4, ntxt, Ttot, gh, gw,
                           attn_mode=0, rope_scale=1.0, bands=None):
    """One rapid-moss step (mossrun.cpp:307-334) with the reference's glue, image by image. z, x0: token rows
    [B][T][C4] (feature c*4 + ph*2 + pw) of a gh x gw grid; returns the new x0. rope_scale: the low-res steps' image
    position scale (mossrun.cpp:313).
    time_vecs (mossrun.cpp:255-264): e = sinusoid_256(code), a = T0 e + b0, b = T2 silu(a) + b2, block modulation
    Wm b + bm [6][D], head modulation Wh b + bh; x_in = z + x0 Q^T per token; rows = Wv x_in + bv, then the text rows
    f16(text Wt^T) (the text projection into zeroed rows); blocks; head RMS(x) nfin (1 + head[D:]) + head[:D],
    v = Wfin r, x0 = z - v.
    glue = (Wv [D][C4], T0 [D][256], T2 [D][D], Wh [2D][D], Wfin [C4][D], Wt [D][ntxt_in]): Wh and Wt fp16, the
    others fp32 or fp16; modw [6D][D] fp16; vec = (bv, b0, b2, bm, bh, nfin, Q [C4][C4], bn_mean, bn_var) fp32;
    bands: the 16 RoPE bands (default 10000^(-i/16))."""
    Wv, T0, T2, Wh, Wfin, Wt = glue
    bv, b0, b2, bm, bh, nfin, Q = vec[:7]
    e = hxo.sinusoid(code, 256)[None, :]
    a = lin(e, T0) + b0
    bt = lin(silu(a), T2) + b2
    mod6 = (hxo.linear_f32(bt, modw)[0] + bm).reshape(6, D).astype(np.float32)
    head = (hxo.linear_f32(bt, Wh)[0] + bh).astype(np.float32)
    if bands is None:
        bands = (1.0 / 10000.0 ** (np.arange(16) / 16.0)).astype(np.float32)
    c, sn = hxo.rope_moss_scaled(gh, gw, ntxt, bands, rope_scale)  # image positions x rope_scale (low-res steps)
    cos = np.ones((Ttot, 64), np.float32)
    sin = np.zeros((Ttot, 64), np.float32)
    cos[:c.shape[0]], sin[:c.shape[0]] = c, sn
    timg = gh * gw
    out = np.zeros_like(x0)
    for b in range(z.shape[0]):
        xin = (z[b].astype(np.float64) + x0[b].astype(np.float64) @ Q.astype(np.float64).T).astype(np.float32)
        x = np.zeros((Ttot, D), np.float32)
        x[:timg] = lin(xin, Wv) + bv
        x[timg:timg + ntxt] = f16(hxo.gemm(txt16[b], Wt)).astype(np.float32)
        for w in blocks:
            x, _, _ = hxo.moss_block(x, mod6, cos, sin, w, H=H, F=F, nvalid=timg + ntxt, attn_mode=attn_mode)
        xi = x[:timg].astype(np.float64)
        rs = 1.0 / np.sqrt((xi * xi).mean(-1, keepdims=True) + 1e-6)
        r = (xi * rs * nfin * (1.0 + head[D:]) + head[:D]).astype(np.float32)
        out[b] = z[b] - lin(r, Wfin)
    return out


def bn_unpatchify(x0, mean, var, Cc, H, W):
    """mossrun.cpp:339-343: x0 token rows [T][4C] (feature c*4 + ph*2 + pw) -> [C][H][W] * sqrt(var + 1e-4) + mean."""
    y = (x0.astype(np.float64) * np.sqrt(var.astype(np.float64) + 1e-4) + mean).astype(np.float32)
    gh, gw = H // 2, W // 2
    return np.ascontiguousarray(y.reshape(gh, gw, Cc, 2, 2).transpose(2, 0, 3, 1, 4).reshape(Cc, H, W))
