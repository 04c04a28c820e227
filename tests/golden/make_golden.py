"""Writes tests/golden/golden.npz: known-answer vectors for the matmul hot path, computed with
exact rational arithmetic (fractions.Fraction) and an explicit IEEE round-to-nearest-even step
at every rounding point the reference defines. Nothing here shares code with the C oracle
(oracle/hi_oracle.c) or with the HIP library: it is the independent side of the oracle's pin.

What the reference fixes, and where:
  quantize_rows     s = fp16(fp32(amax / 127)), q = clamp(round_half_even(fp32(w / s)), +-127),
                    q = 0 when s == 0                         scripts/export.py:54-68
  dequantize_rows   fp16(q * s)                                scripts/export.py:71-73
  gemv / gemm       fp16 of the fp32 dot product; epilogues   src/kernels.cuh:256-264, 454-505
                    residual fp16(out + fp16(y)); SwiGLU fp16(fp16(silu(fp16 g)) * fp16 u)
                    (kernels.cuh:100-105); int8 gemv = (sum q x) * s, int8 gemm on fp16(q s)
  rmsnorm prologue  w * fp16(x * (1 / sqrt(mean x^2 + eps)))  kernels.cuh:182-200
  rope              kernels.cuh:132-136, per-op fp16 rounding
  moe               kernels.cuh:2091-2276, docs/moe-design.md:186-201

Dot products are exact, then rounded once to fp32 (the kernels accumulate in fp32, so the
exact sum rounded once is the ideal fp32 result); exp() comes from math.exp in double, rounded
to fp32, so the SwiGLU and router cases carry a 1-ulp allowance in the tests that read them.

python tests/golden/make_golden.py   (writes golden.npz beside this file; runs in seconds)
"""
import math
import os
import struct
from fractions import Fraction

import numpy as np

HALF = Fraction(1, 2)


def round_bin(x, p, emin, emax):
    """x (Fraction) rounded to nearest-even in a binary format with p significand bits, minimum
    normal exponent emin and maximum exponent emax; returns a Fraction or +-inf (float)."""
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)
    quantum = Fraction(2) ** (e - p + 1)
    n = a / quantum
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > HALF or (rem == HALF and fl % 2 == 1):
        fl += 1
    r = fl * quantum
    if r >= Fraction(2) ** (emax + 1):
        return sign * math.inf
    return sign * r


def f32(x):
    return round_bin(Fraction(x), 24, -126, 127)


def f16(x):
    return round_bin(Fraction(x), 11, -14, 15)


def h_bits(x):
    """fp16 bit pattern of an exactly representable value (Fraction or inf)."""
    return struct.unpack("<H", struct.pack("<e", float(x)))[0]


def f_bits(x):
    return struct.unpack("<I", struct.pack("<f", float(x)))[0]


def h_val(bits):
    return Fraction(struct.unpack("<e", struct.pack("<H", int(bits)))[0])


def rne_int(x):
    fl = x.numerator // x.denominator
    rem = x - fl
    if rem > HALF or (rem == HALF and fl % 2 == 1):
        fl += 1
    return fl


def sqrt_f32(x):
    """Correctly rounded fp32 square root of a positive Fraction (that is itself an fp32 value)."""
    # scale so the integer square root carries far more than 24 bits, then round exactly
    scale = 200
    num = x.numerator << (2 * scale)
    r = math.isqrt(num // x.denominator)
    lo = Fraction(r, 1 << scale) / Fraction(1)  # sqrt(x) in [lo, lo + 2^-scale)
    # the fp32 rounding of sqrt(x) equals that of lo unless lo sits within 2^-scale of a tie;
    # at 200 extra bits that cannot happen for fp32 inputs (sqrt of an fp32 is never a tie)
    return f32(lo)


def silu_mul(g, u):
    """fp32 g, u (Fractions) -> fp16 value (Fraction), kernels.cuh:100-105."""
    gh = f16(g)
    e = f32(Fraction(math.exp(-float(gh))))
    den = f32(1 + e)
    s = f16(f32(gh / den))
    return f16(s * f16(u))


# ------------------------------------------------------------------ quantize_rows
def quantize_row(wbits):
    w = [h_val(b) for b in wbits]
    amax = max(abs(v) for v in w)
    s = f16(f32(amax / 127))
    q = []
    for v in w:
        if s > 0:
            t = rne_int(f32(v / s))
            q.append(max(-127, min(127, t)))
        else:
            q.append(0)
    return q, h_bits(s)


def quant_rows(rng):
    K = 24
    rows = []
    # s = 1: ties at 2.5 / 3.5 / -2.5 / 0.5 / 1.5 go to even
    rows.append([127.0, 2.5, 3.5, -2.5, 0.5, 1.5, -127.0, 0.0, -0.5, 126.5, -3.5, 4.5] + [0.0] * (K - 12))
    rows.append([0.0] * K)  # zero row: s = 0, q = 0
    # subnormal scale: amax 1e-4 -> s = 13 * 2^-24; amax / s = 129.1 -> clamped to 127
    rows.append([1e-4, -1e-4, 5e-5, 2e-6] + [0.0] * (K - 4))
    # scale underflow: amax = 3 * 2^-24 -> amax / 127 below 2^-25 -> s = 0, q = 0
    rows.append([3 * 2.0 ** -24, -(2.0 ** -24)] + [0.0] * (K - 2))
    # an outlier row (few levels for the rest) and a negative-peak row
    r = list(rng.normal(0, 0.02, K)); r[5] = 3.0
    rows.append(r)
    r = list(rng.normal(0, 0.02, K)); r[9] = -0.5
    rows.append(r)
    for _ in range(10):
        rows.append(list(rng.normal(0, 0.02, K)))
    w = np.array(rows, np.float32).astype(np.float16)
    qs, ss = [], []
    for row in w.view(np.uint16):
        q, s = quantize_row(row)
        qs.append(q)
        ss.append(s)
    return w, np.array(qs, np.int8), np.array(ss, np.uint16).view(np.float16)


def dequant(q, s):
    out = np.empty(q.shape, np.uint16)
    for n in range(q.shape[0]):
        sv = h_val(s.view(np.uint16)[n])
        for k in range(q.shape[1]):
            out[n, k] = h_bits(f16(int(q[n, k]) * sv))
    return out.view(np.float16)


# ------------------------------------------------------------------ fp16 conversion KATs
def f16_kats():
    vals = [0.0, -0.0, 1.0, -2.0, 65504.0, 65519.996, 65520.0, 65535.0, 1e9, 2.0 ** -14, 2.0 ** -24, 2.0 ** -25,
            2.0 ** -25 * 1.0000001, 3 * 2.0 ** -25, 5 * 2.0 ** -25, 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11,
            1 + 2.0 ** -11 + 2.0 ** -20, 2.0 ** -14 - 2.0 ** -25, 0.1, -0.3, 1 / 3, 1 / 127]
    f = np.array(vals, np.float32)
    sgn = lambda v: 0x8000 if math.copysign(1.0, float(v)) < 0 else 0  # Fraction drops the sign of -0.0
    h = np.array([(h_bits(f16(Fraction(float(v)))) | sgn(v)) if abs(float(v)) < 65520 else (0x7C00 | sgn(v))
                  for v in f], np.uint16)
    return f, h


# ------------------------------------------------------------------ gemv / gemm
def frac_mat(a):
    return [[Fraction(float(v)) for v in row] for row in np.asarray(a, np.float32)]


def dot(xr, wr):
    return sum((a * b for a, b in zip(xr, wr)), Fraction(0))


def rmsnorm_rows(x, w, eps):
    X, Wn = frac_mat(x), [Fraction(float(v)) for v in np.asarray(w, np.float32)]
    out = []
    K = len(Wn)
    for row in X:
        ss = sum((v * v for v in row), Fraction(0))
        mean = f32(ss / K)
        r = f32(1 / sqrt_f32(f32(mean + f32(Fraction(eps)))))
        out.append([f16(wv * f16(f32(v * r))) for v, wv in zip(row, Wn)])
    return out


def gemv_case(x, W, scales, normw, eps, epi, out0):
    """Known answer of the reference gemv_kernel (src/kernels.cuh:164-281)."""
    X = rmsnorm_rows(x, normw, eps) if normw is not None else frac_mat(x)
    Wr = frac_mat(W.astype(np.float32)) if scales is None else [[Fraction(int(v)) for v in row] for row in W]
    sc = None if scales is None else [h_val(b) for b in scales.view(np.uint16)]
    M, N = len(X), len(Wr)

    def y(m, n):
        d = dot(X[m], Wr[n])
        if sc is not None:
            d = f32(f32(d) * sc[n])  # fp32 sum of q x, times the fp32 scale
        return f32(d)

    n_out = N // 2 if epi == 2 else N
    out = np.empty((M, n_out), np.uint16)
    for m in range(M):
        for o in range(n_out):
            if epi == 0:
                v = f16(y(m, o))
            elif epi == 1:
                v = f16(h_val(out0.view(np.uint16)[m, o]) + f16(y(m, o)))
            else:
                r0 = (o // 16) * 32 + o % 16
                v = silu_mul(y(m, r0), y(m, r0 + 16))
            out[m, o] = h_bits(v)
    return out.view(np.float16)


def gemm_case(A, W, scales, bias, epi, out0):
    """Known answer of the reference gemm_kernel epilogues; int8 weights enter as fp16(q s)."""
    Wh = W if scales is None else dequant(W, scales)
    X, Wr = frac_mat(A), frac_mat(Wh.astype(np.float32))
    M, N = len(X), len(Wr)
    bv = None if bias is None else [Fraction(float(v)) for v in bias.astype(np.float32)]
    n_out = N // 2 if epi == 2 else N
    out = np.empty((M, n_out), np.uint16)
    for m in range(M):
        for o in range(n_out):
            if epi == 0:
                t = f32(dot(X[m], Wr[o]))
                v = f16(f32(t + bv[o]) if bv is not None else t)
            elif epi == 1:
                v = f16(h_val(out0.view(np.uint16)[m, o]) + f16(f32(dot(X[m], Wr[o]))))
            else:
                c = (o // 16) * 32 + o % 16
                v = silu_mul(f32(dot(X[m], Wr[c])), f32(dot(X[m], Wr[c + 16])))
            out[m, o] = h_bits(v)
    return out.view(np.float16)


def qkv_rope_case(x, W, scales, bias, normw, eps, Hq, Hkv, D, cs, pos, max_seq):
    """Known answer of the fused QKV + bias + RoPE + KV write (kernels.cuh:265-278, 132-136)."""
    X = rmsnorm_rows(x, normw, eps) if normw is not None else frac_mat(x)
    Wr = frac_mat(W.astype(np.float32)) if scales is None else [[Fraction(int(v)) for v in row] for row in W]
    sc = None if scales is None else [h_val(b) for b in scales.view(np.uint16)]
    M = len(X)
    HD = D // 2
    out = np.zeros((M, Hq * D), np.uint16)
    kc = np.zeros((M, Hkv, max_seq, D), np.uint16)
    vc = np.zeros((M, Hkv, max_seq, D), np.uint16)
    csb = cs.view(np.uint16)
    for m in range(M):
        p = int(pos[m])
        for head in range(Hq + 2 * Hkv):
            for d in range(HD):
                r0, r1 = head * D + d, head * D + d + HD
                a = []
                for r in (r0, r1):
                    t = dot(X[m], Wr[r])
                    t = f32(f32(t) * sc[r]) if sc is not None else f32(t)
                    if bias is not None:
                        t = f32(t + Fraction(float(bias[r])))
                    a.append(f16(t))
                y1, y2 = a
                if head < Hq + Hkv:
                    c, s = h_val(csb[p, d, 0]), h_val(csb[p, d, 1])
                    y1, y2 = f16(f16(y1 * c) - f16(y2 * s)), f16(f16(y2 * c) + f16(y1 * s))
                if head < Hq:
                    out[m, head * D + d], out[m, head * D + d + HD] = h_bits(y1), h_bits(y2)
                elif head < Hq + Hkv:
                    kc[m, head - Hq, p, d], kc[m, head - Hq, p, d + HD] = h_bits(y1), h_bits(y2)
                else:
                    vc[m, head - Hq - Hkv, p, d], vc[m, head - Hq - Hkv, p, d + HD] = h_bits(y1), h_bits(y2)
    return out.view(np.float16), kc.view(np.float16), vc.view(np.float16)


# ------------------------------------------------------------------ moe
def argmax_better(v, i, best, bi):
    vn, bn = v != v, best != best
    if vn != bn:
        return vn
    return i < bi if (vn or v == best) else v > best


def router_case(xn, Wr, k, flags):
    X, R = frac_mat(xn), frac_mat(Wr)
    M, E = len(X), len(R)
    idx = np.zeros((M, k), np.int32)
    w = np.zeros((M, k), np.float32)
    for t in range(M):
        logit = [float(f16(f32(dot(X[t], R[e])))) for e in range(E)]
        taken = [False] * E
        sel = []
        for _ in range(k):
            best, bi = -math.inf, 1 << 31
            for e in range(E):
                if not taken[e] and argmax_better(logit[e], e, best, bi):
                    best, bi = logit[e], e
            taken[bi] = True
            sel.append((bi, best))
        mx = sel[0][1]
        ex = [f32(Fraction(math.exp(float(f32(Fraction(v) - Fraction(mx)))))) for _, v in sel]
        if flags & 1:
            den = Fraction(0)
            for e_ in ex:
                den = f32(den + e_)
        else:
            den = Fraction(0)
            for e in range(E):
                den = f32(den + f32(Fraction(math.exp(float(f32(Fraction(logit[e]) - Fraction(mx)))))))
        for j, (e, _) in enumerate(sel):
            wj = f32(ex[j] / den)
            if flags & 2:
                wj = f16(wj)
            idx[t, j], w[t, j] = e, float(wj)
    return idx, w


def experts_case(xn, wgu, wdown, idx, w, x0, flags, scale):
    X = frac_mat(xn)
    E, I2, H = wgu.shape
    I = I2 // 2
    M, k = idx.shape
    out = x0.view(np.uint16).copy()
    for t in range(M):
        sums = [Fraction(0)] * H
        for j in range(k):
            e = int(idx[t, j])
            G = frac_mat(wgu[e].astype(np.float32))
            Dn = frac_mat(wdown[e].astype(np.float32))
            act = []
            for i in range(I):
                r0 = (i // 16) * 32 + i % 16
                act.append(silu_mul(f32(dot(X[t], G[r0])), f32(dot(X[t], G[r0 + 16]))))
            wt = Fraction(float(w[t, j]))
            for h in range(H):
                c = f32(f16(f32(dot(act, Dn[h]))) * wt)
                if flags & 2:
                    c = f16(c)
                sums[h] = f32(sums[h] + c)
        for h in range(H):
            o = f16(sums[h])
            if scale != 1.0:
                o = f16(f32(o * Fraction(scale)))
            out[t, h] = h_bits(f16(h_val(out[t, h]) + o))
    return out.view(np.float16)


def main():
    rng = np.random.default_rng(20261201)
    g = {}
    g["f16_in"], g["f16_out"] = f16_kats()
    w, q, s = quant_rows(rng)
    g["quant_w"], g["quant_q"], g["quant_s"] = w, q, s
    g["dequant"] = dequant(q, s)

    h16 = lambda *shape, sd=1.0: (rng.normal(0, sd, shape)).astype(np.float16)
    M, N, K, eps = 3, 64, 48, 1e-5
    x = h16(M, K)
    W = h16(N, K, sd=0.05)
    nw = (rng.random(K) + 0.5).astype(np.float16)
    res = h16(M, N)
    Wq, Ws = quantize_rows_np(W)
    g["gemv_x"], g["gemv_W"], g["gemv_nw"], g["gemv_res"], g["gemv_Wq"], g["gemv_Ws"] = x, W, nw, res, Wq, Ws
    g["gemv_e0"] = gemv_case(x, W, None, None, eps, 0, None)
    g["gemv_e0_norm"] = gemv_case(x, W, None, nw, eps, 0, None)
    g["gemv_e1"] = gemv_case(x, W, None, None, eps, 1, res)
    g["gemv_e2_norm"] = gemv_case(x, W, None, nw, eps, 2, None)
    g["gemv_q_e0"] = gemv_case(x, Wq, Ws, None, eps, 0, None)
    g["gemv_q_e1"] = gemv_case(x, Wq, Ws, None, eps, 1, res)
    g["gemv_q_e2_norm"] = gemv_case(x, Wq, Ws, nw, eps, 2, None)

    bias = h16(N)
    g["gemm_bias"] = bias
    g["gemm_e0_bias"] = gemm_case(x, W, None, bias, 0, None)
    g["gemm_e1"] = gemm_case(x, W, None, None, 1, res)
    g["gemm_e2"] = gemm_case(x, W, None, None, 2, None)
    g["gemm_q_e0"] = gemm_case(x, Wq, Ws, None, 0, None)
    g["gemm_q_e2"] = gemm_case(x, Wq, Ws, None, 2, None)

    Hq, Hkv, D, S = 2, 1, 8, 6
    Kr = 32
    xr = h16(2, Kr)
    Wr = h16((Hq + 2 * Hkv) * D, Kr, sd=0.05)
    br = h16((Hq + 2 * Hkv) * D)
    nwr = (rng.random(Kr) + 0.5).astype(np.float16)
    ang = np.arange(S)[:, None] * (1.0 / 10000 ** (np.arange(0, D, 2) / D))[None, :]
    cs = np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float16)  # [S, D/2, 2]
    pos = np.array([0, 5], np.int32)
    Wrq, Wrs = quantize_rows_np(Wr)
    g.update(rope_x=xr, rope_W=Wr, rope_b=br, rope_nw=nwr, rope_cs=cs, rope_pos=pos, rope_Wq=Wrq, rope_Ws=Wrs)
    o, kc, vc = qkv_rope_case(xr, Wr, None, br, nwr, eps, Hq, Hkv, D, cs, pos, S)
    g.update(rope_out=o, rope_kc=kc, rope_vc=vc)
    o, kc, vc = qkv_rope_case(xr, Wrq, Wrs, None, None, eps, Hq, Hkv, D, cs, pos, S)
    g.update(rope_q_out=o, rope_q_kc=kc, rope_q_vc=vc)

    E, k, H, I = 4, 2, 32, 16
    xn = h16(3, H)
    Wrt = h16(E, H, sd=0.3)
    wgu = h16(E, 2 * I, H, sd=0.1)
    wdn = h16(E, H, I, sd=0.1)
    x0 = h16(3, H)
    g.update(moe_xn=xn, moe_Wr=Wrt, moe_wgu=wgu, moe_wdown=wdn, moe_x0=x0)
    for flags in (1, 2, 3):
        idx, w = router_case(xn, Wrt, k, flags)
        g[f"moe_idx_f{flags}"], g[f"moe_w_f{flags}"] = idx, w
        g[f"moe_out_f{flags}"] = experts_case(xn, wgu, wdn, idx, w, x0, flags, 0.25 if flags == 3 else 1.0)

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")
    np.savez_compressed(path, **g)
    print(f"wrote {path}: {len(g)} arrays")


def quantize_rows_np(W):
    """Quantised weights for the int8 cases, from the exact quantize_row above."""
    qs, ss = [], []
    for row in W.view(np.uint16):
        q, s = quantize_row(row)
        qs.append(q)
        ss.append(s)
    return np.array(qs, np.int8), np.array(ss, np.uint16).view(np.float16)


if __name__ == "__main__":
    main()
