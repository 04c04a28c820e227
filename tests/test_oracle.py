"""Pins the CPU oracle (oracle/hi_oracle.c) before any GPU result is compared with it.

Each oracle function is checked against at least one thing it does not share code with:
  * tests/golden/golden.npz -- exact rational arithmetic with explicit IEEE rounding
    (tests/golden/make_golden.py), bit for bit;
  * library routines the arithmetic reduces to (numpy's float16 conversions, float64 matmul);
  * closed forms and invariants the reference's own tests use (tests/test_int8_cpu.py:95-125,
    tests/test_kernels.py:356-379, 508-518 in the reference checkout).
The cases are chosen so a plausible slip -- a transposed operand, a dropped rounding point, round
half away from zero, a wrong interleave index, a swapped rope sign -- fails at least one of them.
"""
import os

import numpy as np
import pytest

from oracle import oracle as O

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))


def bits(a):
    return np.asarray(a).view(np.uint16)


def ulp_diff(a, b):
    """Distance in fp16 ulps (same-sign finite values)."""
    ia, ib = bits(a).astype(np.int32), bits(b).astype(np.int32)
    ia = np.where(ia & 0x8000, 0x8000 - ia, ia)
    ib = np.where(ib & 0x8000, 0x8000 - ib, ib)
    return np.abs(ia - ib)


# ------------------------------------------------------------------ fp16 conversion
def test_h2f_exhaustive_vs_numpy():
    h = np.arange(65536, dtype=np.uint16)
    got = O.h2f(h.view(np.float16))
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f2h_ties_and_random_vs_numpy():
    # every fp16 value, the fp32 midpoints to its neighbour and one fp32 ulp either side of them
    h = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = (h[:-1] + h[1:]) / 2
    mids = np.concatenate([mids, [65520.0, 2.0 ** -25]]).astype(np.float32)
    around = np.concatenate([mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(0))])
    rng = np.random.default_rng(1)
    rand = rng.integers(0, 2 ** 32, 1 << 21, dtype=np.uint64).astype(np.uint32).view(np.float32)
    f = np.concatenate([around, -around, rand, np.array([np.inf, -np.inf, 1e30, -1e30], np.float32)])
    got = O.f2h(f)
    ref = f.astype(np.float16)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got)[~nan], bits(ref)[~nan])


def test_f2h_golden_kats():
    assert np.array_equal(bits(O.f2h(G["f16_in"])), G["f16_out"])


# ------------------------------------------------------------------ int8 format
def test_quantize_rows_golden():
    q, s = O.quantize_rows(G["quant_w"])
    assert np.array_equal(q, G["quant_q"])
    assert np.array_equal(bits(s), bits(G["quant_s"]))
    # the hand-derived rows: ties to even at s = 1; the subnormal scale clamps to 127; underflow -> 0
    assert q[0, :12].tolist() == [127, 2, 4, -2, 0, 2, -127, 0, 0, 126, -4, 4]
    assert float(s[0]) == 1.0
    assert float(s[1]) == 0.0 and not q[1].any()
    assert bits(s[2]) == 13 and q[2, 0] == 127 and q[2, 1] == -127
    assert float(s[3]) == 0.0 and not q[3].any()


def test_quantize_rows_properties():
    """tests/test_int8_cpu.py:95-107 of the reference: peaks, half-step error, zero rows, chunking."""
    rng = np.random.default_rng(1)
    W = (rng.standard_normal((300, 2048)) * 0.02).astype(np.float16)
    W[7] = 0
    W[9, 5] = 3.0
    q, s = O.quantize_rows(W)
    Wf = W.astype(np.float64)
    nz = np.abs(Wf).max(1) > 0
    peak = np.abs(q.astype(np.int32)).max(1)
    assert (peak[nz] == 127).all() and peak[~nz].max() == 0
    step = s.astype(np.float64)[:, None]
    assert (np.abs(Wf - q * step) <= step * 0.5005).all()
    q1, s1 = O.quantize_rows(W[:123])
    q2, s2 = O.quantize_rows(W[123:])
    assert np.array_equal(np.concatenate([q1, q2]), q) and np.array_equal(bits(np.concatenate([s1, s2])), bits(s))


def test_dequantize_golden_and_exhaustive():
    assert np.array_equal(bits(O.dequantize_rows(G["quant_q"], G["quant_s"])), bits(G["dequant"]))
    # all 256 codes x scales across the fp16 range; q*s is exact in float64, so numpy's
    # correctly rounded float64 -> float16 conversion is the answer
    q = np.tile(np.arange(-128, 128, dtype=np.int16), (8, 1)).astype(np.int8)
    s = np.array([2.0 ** -24, 3 * 2.0 ** -24, 1 / 127, 0.02 / 127, 1.0, 100.0, 255.9, 0.0], np.float16)
    ref = (q.astype(np.float64) * s.astype(np.float64)[:, None]).astype(np.float16)
    assert np.array_equal(bits(O.dequantize_rows(q, s)), bits(ref))


def test_int8_gemv_onehot_kat():
    """Every int8 code at every k position mod 16 comes out exactly (s = 1, x = unit vector):
    the oracle's int8 -> fp32 path is exact (reference tests/test_int8_cpu.py:110-125)."""
    K = 32
    q = np.zeros((256, K), np.int8)
    for v in range(256):
        q[v, v % K] = np.int8(v - 128)
        q[v, (v + 7) % K] = 90  # a neighbour that must not leak in
    s = np.ones(256, np.float16)
    for k in range(K):
        x = np.zeros((1, K), np.float16)
        x[0, k] = 1.0
        out = O.gemv(x, q, scales=s)[0].astype(np.float32)
        assert np.array_equal(out, q[:, k].astype(np.float32))


def test_interleave_matches_reference_formulation():
    """tests/test_kernels.py:35-37 of the reference: stack(view(I/16,16,H) of g and u, 1)."""
    rng = np.random.default_rng(2)
    I, H = 64, 24
    g = rng.standard_normal((I, H)).astype(np.float16)
    u = rng.standard_normal((I, H)).astype(np.float16)
    ref = np.stack([g.reshape(I // 16, 16, H), u.reshape(I // 16, 16, H)], 1).reshape(2 * I, H)
    gu = O.interleave_gate_up(g, u)
    assert np.array_equal(bits(gu), bits(ref))
    assert np.array_equal(bits(gu[16]), bits(u[0])) and np.array_equal(bits(gu[32]), bits(g[16]))
    g2, u2 = O.deinterleave_gate_up(gu)
    assert np.array_equal(bits(g2), bits(g)) and np.array_equal(bits(u2), bits(u))
    qi = O.interleave_gate_up(g.view(np.int16).astype(np.int8), u.view(np.int16).astype(np.int8))
    assert qi.dtype == np.int8 and np.array_equal(qi[16], u.view(np.int16).astype(np.int8)[0])


# ------------------------------------------------------------------ elementwise closed forms
def test_silu_mul_closed_forms():
    assert float(O.silu_mul(0.0, 5.0)) == 0.0
    assert float(O.silu_mul(30.0, 1.0)) == 30.0                # sigmoid(30) rounds to 1
    assert float(O.silu_mul(-30.0, 1.0)) == pytest.approx(0.0, abs=1e-10)
    # silu(g) - silu(-g) = g (odd part), each side within fp16 rounding
    for gv in [0.5, 1.25, 2.0, 3.0]:
        d = float(O.silu_mul(gv, 1.0)) - float(O.silu_mul(-gv, 1.0))
        assert d == pytest.approx(gv, rel=2e-3)
    # the gate is rounded to fp16 before the sigmoid: g and fp16(g) give the same output
    assert bits(O.silu_mul(1.00001, 1.0)) == bits(O.silu_mul(1.0, 1.0))
    # the up value is rounded to fp16 before the product
    assert bits(O.silu_mul(2.0, 1.0 + 2.0 ** -13)) == bits(O.silu_mul(2.0, 1.0))


def test_rmsnorm_closed_form():
    K = 256
    x = np.full((2, K), 0.75, np.float16)
    x[1] = -2.0
    w = np.full(K, 1.5, np.float16)
    y = O.rmsnorm(x, w).astype(np.float64)
    assert np.allclose(y[0], 1.5, rtol=1e-3) and np.allclose(y[1], -1.5, rtol=1e-3)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, K)).astype(np.float16) * 3
    w = (rng.random(K) + 0.5).astype(np.float16)
    xf = x.astype(np.float64)
    ref = w * (xf / np.sqrt((xf ** 2).mean(-1, keepdims=True) + 1e-5))
    assert np.allclose(O.rmsnorm(x, w).astype(np.float64), ref, rtol=2e-3, atol=2e-3)


# ------------------------------------------------------------------ gemv / gemm
GEMV_CASES = [("gemv_e0", dict()), ("gemv_e0_norm", dict(norm=True)), ("gemv_e1", dict(epi=1)),
              ("gemv_e2_norm", dict(epi=2, norm=True)), ("gemv_q_e0", dict(q8=True)), ("gemv_q_e1", dict(q8=True, epi=1)),
              ("gemv_q_e2_norm", dict(q8=True, epi=2, norm=True))]


@pytest.mark.parametrize("name,kw", GEMV_CASES, ids=[c[0] for c in GEMV_CASES])
def test_gemv_golden(name, kw):
    epi = kw.get("epi", 0)
    W, s = (G["gemv_Wq"], G["gemv_Ws"]) if kw.get("q8") else (G["gemv_W"], None)
    out = G["gemv_res"].copy() if epi == 1 else None
    got = O.gemv(G["gemv_x"], W, out=out, normw=G["gemv_nw"] if kw.get("norm") else None, epi=epi, scales=s)
    ref = G[name]
    if epi == 2:  # exp() is libm's in the oracle and math.exp in the generator: 1 ulp allowance
        assert ulp_diff(got, ref).max() <= 1
    else:
        assert np.array_equal(bits(got), bits(ref))


def test_gemv_vs_float64_matmul_and_row_independence():
    rng = np.random.default_rng(4)
    M, N, K = 8, 96, 512
    x = rng.standard_normal((M, K)).astype(np.float16)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float16)
    ref = x.astype(np.float64) @ W.astype(np.float64).T
    got = O.gemv(x, W)
    assert ulp_diff(got, ref.astype(np.float16)).max() <= 1
    # row m of an M-row GEMV equals the 1-row GEMV of that row (api.cu:153-155)
    for m in range(M):
        assert np.array_equal(bits(O.gemv(x[m:m + 1], W)[0]), bits(got[m]))
    # a transposed weight layout would be caught: W^T as [K, N] is not the same product
    assert not np.array_equal(bits(O.gemv(x[:, :96], W[:, :96].T.copy())), bits(got[:, :96]))
    # fp16 one-hot: out[n] = W[n, k] exactly
    for k in [0, 1, 7, 8, 255, 511]:
        e = np.zeros((1, K), np.float16)
        e[0, k] = 1.0
        assert np.array_equal(bits(O.gemv(e, W)[0]), bits(W[:, k]))


GEMM_CASES = [("gemm_e0_bias", dict(bias=True)), ("gemm_e1", dict(epi=1)), ("gemm_e2", dict(epi=2)),
              ("gemm_q_e0", dict(q8=True)), ("gemm_q_e2", dict(q8=True, epi=2))]


@pytest.mark.parametrize("name,kw", GEMM_CASES, ids=[c[0] for c in GEMM_CASES])
def test_gemm_golden(name, kw):
    epi = kw.get("epi", 0)
    W, s = (G["gemv_Wq"], G["gemv_Ws"]) if kw.get("q8") else (G["gemv_W"], None)
    out = G["gemv_res"].copy() if epi == 1 else None
    got = O.gemm(G["gemv_x"], W, out=out, epi=epi, bias=G["gemm_bias"] if kw.get("bias") else None, scales=s)
    if epi == 2:
        assert ulp_diff(got, G[name]).max() <= 1
    else:
        assert np.array_equal(bits(got), bits(G[name]))


def test_gemm_int8_uses_dequantised_weights():
    """int8 GEMM = fp32 math on fp16(q s) (reference tests/test_kernels.py:447), which differs from
    the GEMV's (sum q x) s in the last bits; both stay within tolerance of each other."""
    rng = np.random.default_rng(5)
    A = rng.standard_normal((4, 256)).astype(np.float16)
    q, s = O.quantize_rows((rng.standard_normal((64, 256)) * 0.02).astype(np.float16))
    ref = A.astype(np.float64) @ O.dequantize_rows(q, s).astype(np.float64).T
    assert ulp_diff(O.gemm(A, q, scales=s), ref.astype(np.float16)).max() <= 1
    assert np.allclose(O.gemv(A, q, scales=s).astype(np.float64), ref, rtol=3e-3, atol=3e-3)


@pytest.mark.parametrize("q8", [False, True])
def test_gemv_qkv_rope_golden(q8, ):
    Hq, Hkv, D, S = 2, 1, 8, 6
    M = 2
    out = np.zeros((M, Hq * D), np.float16)
    kc = np.zeros((M, Hkv, S, D), np.float16)
    vc = np.zeros_like(kc)
    if q8:
        O.gemv_qkv_rope(G["rope_x"], G["rope_Wq"], None, Hq, Hkv, G["rope_cs"], G["rope_pos"], kc, vc, out,
                        scales=G["rope_Ws"])
        pre = "rope_q_"
    else:
        O.gemv_qkv_rope(G["rope_x"], G["rope_W"], G["rope_nw"], Hq, Hkv, G["rope_cs"], G["rope_pos"], kc, vc, out,
                        bias=G["rope_b"])
        pre = "rope_"
    assert np.array_equal(bits(out), bits(G[pre + "out"]))
    assert np.array_equal(bits(kc), bits(G[pre + "kc"]))
    assert np.array_equal(bits(vc), bits(G[pre + "vc"]))


def test_rope_closed_forms():
    """Position 0 (cos 1, sin 0) leaves q and k as the plain projection; a quarter turn maps
    (x1, x2) -> (-x2, x1); v is never rotated."""
    rng = np.random.default_rng(6)
    Hq, Hkv, D, K, S = 2, 1, 8, 64, 4
    x = rng.standard_normal((2, K)).astype(np.float16)
    W = (rng.standard_normal(((Hq + 2 * Hkv) * D, K)) * 0.05).astype(np.float16)
    cs = np.zeros((S, D // 2, 2), np.float16)
    cs[0, :, 0] = 1.0
    cs[1, :, 1] = 1.0  # position 1: cos 0, sin 1
    plain = O.gemv(x, W)
    for p, check in [(0, "identity"), (1, "quarter")]:
        out = np.zeros((2, Hq * D), np.float16)
        kc = np.zeros((2, Hkv, S, D), np.float16)
        vc = np.zeros_like(kc)
        O.gemv_qkv_rope(x, W, None, Hq, Hkv, cs, np.array([p, p], np.int32), kc, vc, out)
        qk = np.concatenate([out, kc[:, 0, p]], 1).reshape(2, Hq + Hkv, D)
        ref = plain[:, :(Hq + Hkv) * D].reshape(2, Hq + Hkv, D)
        if check == "identity":
            assert np.array_equal(bits(qk), bits(ref))
        else:
            rot = np.concatenate([-ref[..., D // 2:], ref[..., :D // 2]], -1)
            assert np.array_equal(bits(qk), bits(rot))
        assert np.array_equal(bits(vc[:, 0, p]), bits(plain[:, (Hq + Hkv) * D:]))


# ------------------------------------------------------------------ moe
@pytest.mark.parametrize("flags", [1, 2, 3])
def test_moe_golden(flags):
    idx, w = O.moe_router(G["moe_xn"], G["moe_Wr"], 2, flags)
    assert np.array_equal(idx, G[f"moe_idx_f{flags}"])
    assert np.allclose(w, G[f"moe_w_f{flags}"], rtol=2e-7, atol=0)  # exp(): 1-ulp allowance
    x = G["moe_x0"].copy()
    O.moe_experts(G["moe_xn"], G["moe_wgu"], G["moe_wdown"], G[f"moe_idx_f{flags}"], G[f"moe_w_f{flags}"], x, flags,
                  0.25 if flags == 3 else 1.0)
    assert ulp_diff(x, G[f"moe_out_f{flags}"]).max() <= 1


def test_moe_router_exact_tie_kat():
    """Reference tests/test_kernels.py:508-518: experts 2 and 5 have identical dominant rows ->
    idx [2, 5] (lower index first), weights 1/2 each."""
    rng = np.random.default_rng(7)
    E, k, H = 8, 2, 256
    Wr = (rng.standard_normal((E, H)) * 0.01).astype(np.float16)
    Wr[2] = Wr[5] = 0.05
    xn = (rng.random((4, H)) + 0.5).astype(np.float16)
    idx, w = O.moe_router(xn, Wr, k, 1)
    assert idx.tolist() == [[2, 5]] * 4
    assert np.allclose(w, 0.5, atol=1e-6)


def test_moe_router_order_and_weights():
    rng = np.random.default_rng(8)
    E, k, H = 32, 8, 128
    xn = rng.standard_normal((16, H)).astype(np.float16)
    Wr = (rng.standard_normal((E, H)) * 0.1).astype(np.float16)
    idx, w = O.moe_router(xn, Wr, k, 1)
    logits = (xn.astype(np.float64) @ Wr.astype(np.float64).T).astype(np.float16).astype(np.float64)
    order = np.argsort(-logits, kind="stable", axis=1)[:, :k]
    gap = np.sort(logits, 1)[:, ::-1]
    clear = (gap[:, :k] - gap[:, 1:k + 1]).min(1) > 1e-2
    assert (idx[clear] == order[clear]).all()
    assert np.allclose(w.sum(1), 1.0, atol=1e-5) and (np.diff(w, axis=1) <= 0).all()
    _, w_all = O.moe_router(xn, Wr, k, 0)  # softmax over all E: weights sum below 1
    assert (w_all.sum(1) < 1.0).all()


def test_moe_experts_vs_dense_float64():
    """The routed experts equal a dense float64 formulation (every expert computed, then the
    top-k picked) to fp16 tolerance."""
    rng = np.random.default_rng(9)
    M, E, k, H, I = 5, 8, 2, 64, 32
    xn = rng.standard_normal((M, H)).astype(np.float16)
    Wr = (rng.standard_normal((E, H)) * 0.2).astype(np.float16)
    wgu = (rng.standard_normal((E, 2 * I, H)) * 0.05).astype(np.float16)
    wdn = (rng.standard_normal((E, H, I)) * 0.05).astype(np.float16)
    x0 = rng.standard_normal((M, H)).astype(np.float16)
    idx, w = O.moe_router(xn, Wr, k, 1)
    x = x0.copy()
    O.moe_experts(xn, wgu, wdn, idx, w, x, 1, 1.0)
    xf = xn.astype(np.float64)
    ref = x0.astype(np.float64)
    for t in range(M):
        for j in range(k):
            e = idx[t, j]
            g, u = O.deinterleave_gate_up(wgu[e])
            gg, uu = xf[t] @ g.astype(np.float64).T, xf[t] @ u.astype(np.float64).T
            act = gg / (1 + np.exp(-gg)) * uu
            ref[t] += w[t, j] * (act @ wdn[e].astype(np.float64).T)
    assert np.allclose(x.astype(np.float64), ref, rtol=1e-2, atol=1e-2)


def _np_decode_attn(q, kc, vc, pos, Hq, Hkv):
    """Independent float64 restatement (numpy, the reference's ref_attn form, tests/test_kernels.py:298-307)."""
    B, _, S, D = kc.shape
    G = Hq // Hkv
    out = np.empty((B, Hq * D))
    for b in range(B):
        L = pos[b] + 1
        qb = q[b].astype(np.float64).reshape(Hq, D)
        k = np.repeat(kc[b, :, :L].astype(np.float64), G, axis=0)  # [Hq, L, D]
        v = np.repeat(vc[b, :, :L].astype(np.float64), G, axis=0)
        s = np.einsum("hd,hld->hl", qb, k) / np.sqrt(D)
        p = np.exp(s - s.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        out[b] = np.einsum("hl,hld->hd", p, v).reshape(-1)
    return out


def test_decode_attn_closed_forms():
    """One key: the output is that key's value row (softmax of one logit is 1). Identical keys or a
    zero query: uniform weights, the mean of the values. The kv head of query head h is h / G."""
    r = np.random.default_rng(30)
    B, Hkv, G, S, D = 2, 3, 2, 40, 64
    Hq = Hkv * G
    kc = (r.standard_normal((B, Hkv, S, D))).astype(np.float16)
    vc = (r.standard_normal((B, Hkv, S, D))).astype(np.float16)
    q = r.standard_normal((B, Hq * D)).astype(np.float16)
    out = O.decode_attn(q, kc, vc, np.zeros(B, np.int32), Hq, Hkv)
    for b in range(B):
        for h in range(Hq):
            assert np.array_equal(out[b, h * D:(h + 1) * D], vc[b, h // G, 0]), (b, h)
    pos = np.array([17, 39], np.int32)
    out = O.decode_attn(np.zeros_like(q), kc, vc, pos, Hq, Hkv)
    for b in range(B):
        for h in range(Hq):
            mean = vc[b, h // G, :pos[b] + 1].astype(np.float64).mean(0)
            assert np.array_equal(out[b, h * D:(h + 1) * D], mean.astype(np.float32).astype(np.float16)), (b, h)
    kc2 = np.repeat(kc[:, :, :1], S, axis=2)
    out = O.decode_attn(q, kc2, vc, pos, Hq, Hkv)
    out0 = O.decode_attn(np.zeros_like(q), kc, vc, pos, Hq, Hkv)
    assert np.array_equal(out, out0)


def test_decode_attn_vs_numpy_float64():
    r = np.random.default_rng(31)
    for B, Hkv, G, S, D in [(3, 2, 4, 300, 128), (2, 4, 1, 100, 64), (1, 1, 7, 513, 128)]:
        Hq = Hkv * G
        kc = r.standard_normal((B, Hkv, S, D)).astype(np.float16)
        vc = r.standard_normal((B, Hkv, S, D)).astype(np.float16)
        q = r.standard_normal((B, Hq * D)).astype(np.float16)
        pos = r.integers(0, S, B).astype(np.int32)
        got = O.decode_attn(q, kc, vc, pos, Hq, Hkv).astype(np.float64)
        ref = _np_decode_attn(q, kc, vc, pos, Hq, Hkv)
        # fp16 rounding of a float64 value: half an ulp of fp16 (2^-11 relative), plus the tiny
        # difference in summation order
        assert np.all(np.abs(got - ref) <= 2.0 ** -11 * np.abs(ref) + 1e-7), (B, Hkv, G, S, D)


def test_argmax_matches_numpy_and_edge_rows():
    """The reference's argmax cases (tests/test_kernels.py:208-221): ties to the lowest index, NaN
    wins, a row of -inf or of NaN gives 0, +inf; numpy's argmax has the same rules."""
    r = np.random.default_rng(32)
    V = 32000
    lg = r.standard_normal((8, V)).astype(np.float16)
    lg[1, 100] = lg[1, 31999] = 20.0
    lg[2, 5000] = np.nan
    lg[2, 7] = np.nan
    lg[3] = -np.inf
    lg[4] = np.nan
    lg[5, 31999] = np.inf
    lg[6, 17] = lg[6, 12] = lg[6, 30000] = 60000.0
    lg[7] = 0.0
    got = O.argmax(lg)
    assert np.array_equal(got, np.argmax(lg, -1).astype(np.int32)), got
    assert list(got[[1, 3, 4, 6, 7]]) == [100, 0, 0, 12, 0]


# ------------------------------------------------------------------ prefill: rope_cache, flash_prefill
def test_rope_cache_matches_golden_pinned_qkv_rope():
    """rope_cache on a qkv row equals gemv_qkv_rope (pinned bit for bit by the golden vectors above)
    with identity weights, whose projection is the row itself (one exact product per output), in
    both the decode form (per-row positions and slots) and the prefill form (pos_base + m in one
    slot); v is copied, never rotated."""
    r = np.random.default_rng(40)
    for Hq, Hkv, D in [(4, 2, 64), (3, 1, 128)]:
        S, M = 300, 3
        nh = Hq + 2 * Hkv
        ang = np.arange(S)[:, None] * (1.0 / 10000.0 ** (np.arange(0, D, 2) / D))[None, :]
        cs = np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float16)
        x = r.standard_normal((M, nh * D)).astype(np.float16)
        eye = np.eye(nh * D, dtype=np.float16)
        pos = np.array([7, 299, 0], np.int32)
        out = np.zeros((M, Hq * D), np.float16)
        kc_ref = np.zeros((M, Hkv, S, D), np.float16)
        vc_ref = np.zeros_like(kc_ref)
        O.gemv_qkv_rope(x, eye, None, Hq, Hkv, cs, pos, kc_ref, vc_ref, out)
        qkv = x.copy()
        kc, vc = np.zeros_like(kc_ref), np.zeros_like(vc_ref)
        O.rope_cache(qkv, Hq, Hkv, cs, kc, vc, pos=pos)
        assert np.array_equal(bits(qkv[:, :Hq * D]), bits(out))
        assert np.array_equal(bits(qkv[:, Hq * D:]), bits(x[:, Hq * D:])), "k/v columns must stay as they were"
        assert np.array_equal(bits(kc), bits(kc_ref)) and np.array_equal(bits(vc), bits(vc_ref))
        # prefill form: rows at positions p0..p0+M-1 of slot 1
        p0 = 100
        qkv = x.copy()
        kc, vc = np.zeros((2, Hkv, S, D), np.float16), np.zeros((2, Hkv, S, D), np.float16)
        O.rope_cache(qkv, Hq, Hkv, cs, kc, vc, pos_base=p0, slot_base=1)
        for m in range(M):
            o1 = np.zeros((1, Hq * D), np.float16)
            k1, v1 = np.zeros((1, Hkv, S, D), np.float16), np.zeros((1, Hkv, S, D), np.float16)
            O.gemv_qkv_rope(x[m:m + 1], eye, None, Hq, Hkv, cs, np.array([p0 + m], np.int32), k1, v1, o1)
            assert np.array_equal(bits(qkv[m, :Hq * D]), bits(o1[0]))
            assert np.array_equal(bits(kc[1, :, p0 + m]), bits(k1[0, :, p0 + m]))
            assert np.array_equal(bits(vc[1, :, p0 + m]), bits(v1[0, :, p0 + m]))
        assert not kc[0].any() and not vc[0].any(), "slot 0 untouched"


def test_flash_prefill_rows_are_decode_attention():
    """Row t of a prefill is decode attention at position p0 + t over the same slot (decode_attn is
    pinned by closed forms and numpy above), bit for bit; T = 1 at p0 = 0 returns the first value
    row; a zero query gives the prefix mean; lse of a zero query is log2 of the key count."""
    r = np.random.default_rng(41)
    for Hq, Hkv, D, T, p0 in [(8, 2, 64, 37, 0), (6, 6, 128, 20, 50), (7, 1, 128, 5, 300)]:
        S = p0 + T + 3
        q = r.standard_normal((T, Hq * D)).astype(np.float16)
        kc = r.standard_normal((Hkv, S, D)).astype(np.float16)
        vc = r.standard_normal((Hkv, S, D)).astype(np.float16)
        got, lse = O.flash_prefill(q, kc, vc, T, p0, Hq, Hkv, lse=True)
        dec = O.decode_attn(q, np.broadcast_to(kc, (T,) + kc.shape).copy(), np.broadcast_to(vc, (T,) + vc.shape).copy(),
                            np.arange(p0, p0 + T, dtype=np.int32), Hq, Hkv)
        assert np.array_equal(bits(got), bits(dec)), (Hq, Hkv, D, T, p0)
        # lse against numpy: log2 sum 2^(s log2 e / sqrt D)
        G = Hq // Hkv
        for t in [0, T - 1]:
            for h in [0, Hq - 1]:
                s = kc[h // G, :p0 + t + 1].astype(np.float64) @ q[t, h * D:(h + 1) * D].astype(np.float64) / np.sqrt(D)
                ref = np.log2(np.exp(s - s.max()).sum()) + s.max() / np.log(2)
                assert abs(lse[h, t] - ref) <= 1e-5 * max(1.0, abs(ref)), (t, h, lse[h, t], ref)
        z, lz = O.flash_prefill(np.zeros_like(q), kc, vc, T, p0, Hq, Hkv, lse=True)
        for t in [0, T // 2, T - 1]:
            mean = vc[:, :p0 + t + 1].astype(np.float64).mean(1)  # [Hkv, D]
            assert np.array_equal(z[t].reshape(Hq, D), np.repeat(mean, G, 0).astype(np.float32).astype(np.float16))
            assert np.allclose(lz[:, t], np.log2(p0 + t + 1), rtol=0, atol=1e-6)
    one = O.flash_prefill(q[:1], kc, vc, 1, 0, Hq, Hkv)
    assert np.array_equal(one.reshape(Hq, -1), np.repeat(vc[:, 0], Hq // Hkv, 0))


def test_flash_prefill_vs_numpy_float64_causal():
    """Against a float64 numpy restatement of the reference's ref_attn (tests/test_kernels.py:288-296):
    softmax over the causal mask key <= p0 + t."""
    r = np.random.default_rng(42)
    Hq, Hkv, D, T, p0 = 4, 2, 64, 29, 13
    S = 64
    q = r.standard_normal((T, Hq * D)).astype(np.float16)
    kc = r.standard_normal((Hkv, S, D)).astype(np.float16)
    vc = r.standard_normal((Hkv, S, D)).astype(np.float16)
    got = O.flash_prefill(q, kc, vc, T, p0, Hq, Hkv).astype(np.float64)
    G = Hq // Hkv
    k = np.repeat(kc[:, :p0 + T].astype(np.float64), G, 0)
    v = np.repeat(vc[:, :p0 + T].astype(np.float64), G, 0)
    s = np.einsum("thd,hld->htl", q.astype(np.float64).reshape(T, Hq, D), k) / np.sqrt(D)
    s[:, np.arange(p0 + T)[None, :] > (p0 + np.arange(T))[:, None]] = -np.inf
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    ref = np.einsum("htl,hld->thd", p, v).reshape(T, Hq * D)
    assert np.all(np.abs(got - ref) <= 2.0 ** -11 * np.abs(ref) + 1e-7)
