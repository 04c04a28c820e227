"""GPU parity of the decode GEMV and the int8 quantiser, through the C-ABI (hipinfer_amd.hipinfer),
against the CPU oracle on the same seeded inputs.

Mirrors the reference's tests/test_kernels.py test_gemv (47-65), test_gemv_qkv_rope (264-286),
test_quantize_rows (364-379) and test_gemv_int8 (382-440): same shapes, row counts and
tolerances, with the oracle (oracle/hi_oracle.c) in place of torch's fp32 math. Adds the checks
the MI355X design needs: exact int8 unpacking for every code at every lane position, row
independence (row m of an M-row GEMV equals the 1-row GEMV bit for bit), the 8-byte int8 path
(K % 16 == 8), row chunking (M = 16 at large K), strided activations/outputs, and argument
rejection.
"""
import numpy as np
import pytest

from tests._util import bits, check, cuda, gpu, h16, host, interleave, rng

pytestmark = gpu


@pytest.fixture(scope="module")
def hi():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from hipinfer_amd import hipinfer
    return hipinfer


@pytest.fixture(scope="module")
def O():
    from oracle import oracle
    return oracle


def q8(O, W):
    return O.quantize_rows(W)


SHAPES = [(2048, 5632), (896, 4864), (3072, 8192)]


@pytest.mark.parametrize("H,I", SHAPES)
@pytest.mark.parametrize("q", [False, True], ids=["fp16", "int8"])
def test_gemv_epilogues(hi, O, H, I, q):
    r = rng(100 + H)
    for M in [1, 3, 8, 11]:
        x = h16(r, M, H)
        W = h16(r, 2560, H, sd=0.02)
        s = None
        if q:
            W, s = q8(O, W)
        got = host(hi.gemv(cuda(x), cuda(W), scales=None if s is None else cuda(s)))
        check(f"gemv M={M} K={H}", got, O.gemv(x, W, scales=s), 2e-3, 2e-3)
        nw = (r.random(H) + 0.5).astype(np.float16)
        got = host(hi.gemv(cuda(x), cuda(W), normw=cuda(nw), scales=None if s is None else cuda(s)))
        check(f"gemv+rmsnorm M={M} K={H}", got, O.gemv(x, W, normw=nw, scales=s), 3e-3, 3e-3)
        res = h16(r, M, H)
        W2 = h16(r, H, I, sd=0.02)
        s2 = None
        if q:
            W2, s2 = q8(O, W2)
        a = h16(r, M, I)
        out = cuda(res)
        hi.gemv(cuda(a), cuda(W2), out=out, epi=1, scales=None if s2 is None else cuda(s2))
        check(f"gemv+residual M={M} K={I}", host(out), O.gemv(a, W2, out=res.copy(), epi=1, scales=s2), 4e-3, 2e-3)
        gu = interleave(h16(r, I, H, sd=0.02), h16(r, I, H, sd=0.02))
        sg = None
        if q:
            gu, sg = q8(O, gu)
        got = host(hi.gemv(cuda(x), cuda(gu), epi=2, normw=cuda(nw), scales=None if sg is None else cuda(sg)))
        check(f"gemv+norm+swiglu M={M} I={I}", got, O.gemv(x, gu, epi=2, normw=nw, scales=sg), 3e-3, 3e-3)


@pytest.mark.parametrize("q", [False, True], ids=["fp16", "int8"])
def test_every_row_written_across_grid_shapes(hi, O, q):
    """The launch deals units to k blocks per CU with ipb items each (fewer items than CUs: one block
    per item; partial last rounds; ipb below 8). Over unit counts that exercise each case, every
    output row is written (the output starts as NaN) and matches the oracle."""
    import torch
    r = rng(7)
    K = 256
    for N in [1, 17, 100, 255, 256, 257, 700, 2047, 3000, 5000, 9000]:
        for M in [1, 5]:
            x = h16(r, M, K)
            W = h16(r, N, K, sd=0.02)
            s = None
            if q:
                W, s = q8(O, W)
            out = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
            hi.gemv(cuda(x), cuda(W), out=out, scales=None if s is None else cuda(s))
            got = host(out)
            assert np.isfinite(got.astype(np.float32)).all(), f"N={N} M={M}: rows left unwritten"
            check(f"N={N} M={M}", got, O.gemv(x, W, scales=s), 2e-3, 2e-3)


@pytest.mark.parametrize("K,ks", [(64 * 16 * 2, [0, 1, 2, 3, 5, 8, 13, 15, 16, 17, 1023, 1024, 2047]),
                                   (1536, [0, 15, 1023, 1024, 1031, 1032, 1039, 1535])],
                         ids=["K2048", "K1536"])
def test_int8_unpack_every_code_every_position(hi, K, ks):
    """Each int8 code at each of the 16 byte positions of a 16-byte load (and across the 64
    lanes) comes out exactly: s = 1, x = a unit vector -> out[n] = q[n, k]. K = 1536 (96 chunks a
    row) ends in a slot of 64 lanes that only half fill."""
    import torch
    q = np.zeros((256, K), np.int8)
    for v in range(256):
        q[v, :] = np.int8(((v * 37) % 255) - 127)  # neighbours that must not leak in
    for k in ks:
        qq = q.copy()
        qq[:, k] = (np.arange(256) - 128).astype(np.int8)
        x = np.zeros((1, K), np.float16)
        x[0, k] = 1.0
        out = host(hi.gemv(cuda(x), cuda(qq), scales=torch.ones(256, dtype=torch.float16, device="cuda")))
        assert np.array_equal(out[0].astype(np.float32), qq[:, k].astype(np.float32)), f"k={k}"


def test_fp16_onehot_exact(hi):
    r = rng(7)
    K = 4096
    W = h16(r, 300, K, sd=0.5)
    for k in [0, 7, 8, 511, 512, 4095]:
        x = np.zeros((1, K), np.float16)
        x[0, k] = 1.0
        assert np.array_equal(bits(host(hi.gemv(cuda(x), cuda(W)))[0]), bits(W[:, k]))


@pytest.mark.parametrize("q", [False, True], ids=["fp16", "int8"])
@pytest.mark.parametrize("norm", [False, True], ids=["plain", "norm"])
@pytest.mark.parametrize("H", [2048, 1536])
def test_row_independence(hi, O, q, norm, H):
    """Row m of an M-row GEMV is bit-identical to the 1-row GEMV of that row (reference
    api.cu:153-155), for every M the launcher chunks differently; K = 1536 (the C4 hidden size)
    leaves the last 64-lane slot of a row half full."""
    r = rng(8)
    N = 1024
    x = h16(r, 16, H)
    W = h16(r, N, H, sd=0.02)
    s = None
    if q:
        W, s = q8(O, W)
    Wd, sd = cuda(W), None if s is None else cuda(s)
    nw = cuda((r.random(H) + 0.5).astype(np.float16)) if norm else None
    ones = [host(hi.gemv(cuda(x[m:m + 1]), Wd, normw=nw, scales=sd))[0] for m in range(16)]
    for M in ([2, 3, 5, 6, 7, 8] if norm else [2, 3, 5, 6, 7, 8, 16]):
        got = host(hi.gemv(cuda(x[:M]), Wd, normw=nw, scales=sd))
        for m in range(M):
            assert np.array_equal(bits(got[m]), bits(ones[m])), f"M={M} row {m}"


# (D, Hq, Hkv, K, bias): TinyLlama, Llama-3.2-3B, Qwen2.5-1.5B (C4, with bias), a 14-head shape,
# and Llama-3.1-8B (C2: 32 q heads, 8 kv heads, head_dim 128, K = 4096)
QKV = [(64, 32, 4, 2048, False), (128, 24, 8, 3072, False), (128, 12, 2, 1536, True), (64, 14, 2, 896, True),
       (128, 32, 8, 4096, False)]


def rope_table(S, D, theta=10000.0):
    inv = 1.0 / (theta ** (np.arange(0, D, 2, dtype=np.float64) / D))
    ang = np.arange(S)[:, None] * inv[None, :]
    return np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float16)  # [S, D/2, 2]


@pytest.mark.parametrize("D,Hq,Hkv,H,bias", QKV)
@pytest.mark.parametrize("q", [False, True], ids=["fp16", "int8"])
def test_gemv_qkv_rope(hi, O, D, Hq, Hkv, H, bias, q):
    r = rng(200 + D + Hq)
    S = 512
    cs = rope_table(S, D)
    for M in [1, 3, 6, 8]:
        x = h16(r, M, H)
        W = h16(r, (Hq + 2 * Hkv) * D, H, sd=0.02)
        s = None
        if q:
            W, s = q8(O, W)
        b = h16(r, (Hq + 2 * Hkv) * D) if bias else None
        nw = (r.random(H) + 0.5).astype(np.float16)
        pos = r.integers(0, S, M).astype(np.int32)
        out_r = np.zeros((M, Hq * D), np.float16)
        kc_r = np.zeros((M, Hkv, S, D), np.float16)
        vc_r = np.zeros_like(kc_r)
        O.gemv_qkv_rope(x, W, nw, Hq, Hkv, cs, pos, kc_r, vc_r, out_r, bias=b, scales=s)
        out = cuda(np.zeros((M, Hq * D), np.float16))
        kc, vc = cuda(np.zeros_like(kc_r)), cuda(np.zeros_like(vc_r))
        hi.gemv_qkv_rope(cuda(x), cuda(W), cuda(nw), Hq, Hkv, cuda(cs), cuda(pos), kc, vc, out,
                         bias=None if b is None else cuda(b), scales=None if s is None else cuda(s))
        tag = f"D={D} G={Hq // Hkv}{' bias' if bias else ''} M={M}"
        # the two sums differ in order: allow 1 fp16 ulp before the rotation (reference tolerance)
        check(f"qkv+rope {tag}: q", host(out), out_r, 2e-2, 2e-3)
        check(f"qkv+rope {tag}: k cache", host(kc), kc_r, 2e-2, 2e-3)
        check(f"qkv+rope {tag}: v cache", host(vc), vc_r, 2e-2, 2e-3)


def test_quantize_rows_bit_exact(hi, O):
    """GPU quantiser == oracle == exact-arithmetic golden rows (reference export.py:54-68)."""
    import os
    G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))
    q, s = hi.quantize_rows(cuda(G["quant_w"]))
    assert np.array_equal(host(q), G["quant_q"]) and np.array_equal(bits(host(s)), bits(G["quant_s"]))
    assert np.array_equal(bits(host(hi.dequantize_rows(q, s))), bits(G["dequant"]))
    r = rng(9)
    for N, K in [(300, 2048), (64, 4100), (17, 7)]:
        W = h16(r, N, K, sd=0.02)
        W[min(7, N - 1)] = 0
        W[0, min(5, K - 1)] = 3.0
        qg, sg = hi.quantize_rows(cuda(W))
        qo, so = O.quantize_rows(W)
        assert np.array_equal(host(qg), qo) and np.array_equal(bits(host(sg)), bits(so)), f"N={N} K={K}"
        assert np.array_equal(bits(host(hi.dequantize_rows(qg, sg))), bits(O.dequantize_rows(qo, so)))


def test_int8_rows_of_8_byte_alignment(hi, O):
    """K % 16 == 8: rows are only 8-byte aligned, the 8-byte load path runs."""
    r = rng(10)
    for K in [8, 24, 1000, 4104]:
        x = h16(r, 3, K)
        W, s = q8(O, h16(r, 320, K, sd=0.02))
        got = host(hi.gemv(cuda(x), cuda(W), scales=cuda(s)))
        check(f"int8 K={K}", got, O.gemv(x, W, scales=s), 2e-3, 2e-3)


def test_strides_chunking_and_odd_sizes(hi, O):
    import torch
    r = rng(11)
    # strided activations and outputs
    x = h16(r, 5, 1024 + 64)
    W = h16(r, 777, 1024, sd=0.02)
    xd = cuda(x)[:, :1024]
    out = torch.zeros(5, 800, dtype=torch.float16, device="cuda")
    hi.gemv(xd, cuda(W), out=out[:, :777])
    check("strided x/out", host(out[:, :777]), O.gemv(np.ascontiguousarray(x[:, :1024]), W), 2e-3, 2e-3)
    assert not host(out[:, 777:]).any(), "wrote past N"
    # M = 16 rows at a K where 16 rows exceed LDS: the launcher chunks the rows
    x = h16(r, 16, 14336)
    W, s = q8(O, h16(r, 96, 14336, sd=0.02))
    check("M=16 K=14336 int8", host(hi.gemv(cuda(x), cuda(W), scales=cuda(s))), O.gemv(x, W, scales=s), 2e-3, 2e-3)
    # minimum K and a single output row
    x = h16(r, 2, 8)
    W = h16(r, 1, 8)
    check("K=8 N=1", host(hi.gemv(cuda(x), cuda(W))), O.gemv(x, W), 2e-3, 2e-3)


def test_max_smem_bounds_the_activation_rows(hi, O):
    """hi_max_smem (the reference's api.cu:49) reports the LDS a block may opt into. The GEMV stages
    its activation rows there: rows that do not fit together run in chunks (each row unchanged, checked
    against the oracle), and a single row longer than the LDS is refused cleanly."""
    import torch
    lim = hi.lib.hi_max_smem()
    assert lim >= 64 * 1024 and lim % 1024 == 0, lim
    r = rng(31)
    K = (lim // 2 // 8 - 640) * 8  # one row fits, sixteen do not
    assert 16 * K * 2 > lim
    x, W = h16(r, 16, K), (r.standard_normal((32, K)) * 0.02).astype(np.float16)
    check("16 rows in chunks", host(hi.gemv(cuda(x), cuda(W))), O.gemv(x, W), 3e-3, 3e-3)
    K = (lim // 2 // 8 + 8) * 8  # one row alone is longer than the LDS
    with pytest.raises(Exception):
        hi.gemv(torch.zeros(1, K, dtype=torch.float16, device="cuda"), torch.zeros(16, K, dtype=torch.float16, device="cuda"))


def test_rows_per_launch(hi):
    """hi_gemv_rows_per_launch: 8 rows with the fused norm and 16 without while they fit the LDS,
    halved until they do (the Llama-3.1-8B down projection's 28 KB rows: 4), 0 for a row longer
    than the LDS; the launcher's row chunks follow it (checked above at M = 16, K = 14336)."""
    lim = hi.lib.hi_max_smem()
    f = hi.lib.hi_gemv_rows_per_launch
    assert f(4096, 1, 0) == 8 and f(4096, 0, 0) == 16 and f(1536, 0, 1) == 16
    assert f(14336, 0, 0) == 4 and f(14336, 0, 1) == 4
    assert f((lim // 2 // 8 + 8) * 8, 0, 0) == 0


def test_rejects_bad_arguments(hi):
    import torch
    x = torch.zeros(1, 12, dtype=torch.float16, device="cuda")
    W = torch.zeros(4, 12, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        hi.gemv(x, W)  # K % 8 != 0
    x = torch.zeros(1, 64, dtype=torch.float16, device="cuda")
    W = torch.zeros(48, 64, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        hi.gemv(x, W, epi=2)  # SwiGLU needs N % 32 == 0
    with pytest.raises(ValueError):
        hi.gemv(x, W, epi=5)


def test_full_size_sampled_rows(hi, O):
    """Llama-3.1-8B gate/up (28672 x 4096, fused norm + SwiGLU) and lm_head-sized shapes at full
    size: 256 sampled output units checked against the oracle, plus row independence."""
    import torch
    r = rng(12)
    H, I = 4096, 14336
    g = torch.Generator(device="cuda").manual_seed(12)
    W = (torch.randn(2 * I, H, generator=g, device="cuda") * 0.02).half()
    x = h16(r, 1, H)
    nw = (r.random(H) + 0.5).astype(np.float16)
    for q in [False, True]:
        Wd, sd = (W, None) if not q else hi.quantize_rows(W)
        got = host(hi.gemv(cuda(x), Wd, epi=2, normw=cuda(nw), scales=sd))
        units = np.sort(r.choice(I, 256, replace=False))
        rows = np.concatenate([(units // 16) * 32 + units % 16, (units // 16) * 32 + units % 16 + 16])
        Wh = host(Wd[torch.from_numpy(rows).cuda()])
        sh = None if sd is None else host(sd[torch.from_numpy(rows).cuda()])
        # the sampled units as a 256-unit interleaved matrix of their own
        blk = np.empty((512,) + Wh.shape[1:], Wh.dtype)
        sblk = None if sh is None else np.empty(512, np.float16)
        for i in range(256):
            j = (i // 16) * 32 + i % 16
            blk[j], blk[j + 16] = Wh[i], Wh[256 + i]
            if sblk is not None:
                sblk[j], sblk[j + 16] = sh[i], sh[256 + i]
        ref = O.gemv(x, blk, epi=2, normw=nw, scales=sblk)
        check(f"full-size gate/up {'int8' if q else 'fp16'} sampled", got[:, units], ref, 3e-3, 3e-3)


@pytest.mark.parametrize("q", [False, True], ids=["fp16", "int8"])
def test_grouped_units_lm_head_sized(hi, O, q):
    """From 4 rows on, lm_head-sized launches let one wave stream 2 (fp16) or 4 (int8) output rows
    at once. N = 32775 leaves a partial last group. Every activation row must stay bit-identical to
    the 1-row GEMV (one row per wave), for the plain, fused-norm and residual epilogues, and
    sampled output columns must match the oracle."""
    import torch
    r = rng(21)
    N, K = 32775, 1536
    g = torch.Generator(device="cuda").manual_seed(21)
    Wd = (torch.randn(N, K, generator=g, device="cuda") * 0.02).half()
    sd = None
    if q:
        Wd, sd = hi.quantize_rows(Wd)
    x = h16(r, 16, K)
    nw = (r.random(K) + 0.5).astype(np.float16)
    cols = np.concatenate([np.sort(r.choice(N - 8, 120, replace=False)), np.arange(N - 8, N)])
    Wh = host(Wd[torch.from_numpy(cols).cuda()])
    sh = None if sd is None else host(sd[torch.from_numpy(cols).cuda()])
    for norm in [False, True]:
        nwd = cuda(nw) if norm else None
        ones = [host(hi.gemv(cuda(x[m:m + 1]), Wd, normw=nwd, scales=sd))[0] for m in range(16)]
        for M in ([4, 5, 6, 7, 8] if norm else [4, 5, 6, 7, 8, 16]):
            got = host(hi.gemv(cuda(x[:M]), Wd, normw=nwd, scales=sd))
            for m in range(M):
                assert np.array_equal(bits(got[m]), bits(ones[m])), f"norm={norm} M={M} row {m}"
            ref = O.gemv(x[:M], Wh, normw=nw if norm else None, scales=sh)
            check(f"grouped {'int8' if q else 'fp16'} norm={norm} M={M} sampled", got[:, cols], ref, 3e-3, 3e-3)
    # residual epilogue: out = res + x @ W^T, bit-identical per row to the 1-row call
    res = h16(r, 8, N)
    ones = []
    for m in range(8):
        o = cuda(res[m:m + 1])
        hi.gemv(cuda(x[m:m + 1]), Wd, out=o, epi=1, scales=sd)
        ones.append(host(o)[0])
    o = cuda(res)
    hi.gemv(cuda(x[:8]), Wd, out=o, epi=1, scales=sd)
    got = host(o)
    for m in range(8):
        assert np.array_equal(bits(got[m]), bits(ones[m])), f"residual row {m}"
    ref = O.gemv(x[:8], Wh, out=res[:, cols].copy(), epi=1, scales=sh)
    check(f"grouped {'int8' if q else 'fp16'} residual sampled", got[:, cols], ref, 4e-3, 2e-3)


def gpu_weights(hi, seed, N, K, q):
    """[N, K] weights ~N(0, 0.02) generated on the GPU (lm_head-sized matrices), int8-quantised on the
    GPU when q (the quantiser is bit-exact against the oracle, test_quantize_rows_bit_exact)."""
    import torch
    g = torch.Generator(device="cuda").manual_seed(seed)
    W = (torch.randn(N, K, generator=g, device="cuda") * 0.02).half()
    return (W, None) if not q else hi.quantize_rows(W)


def sampled_lm_head(hi, O, r, Wd, sd, x, nw, name):
    """Fused-norm lm_head GEMV at full size; 248 sampled columns plus the last 8 against the oracle
    (columns are independent, so the oracle's GEMV over the sampled rows is exact for them)."""
    import torch
    N = Wd.shape[0]
    got = host(hi.gemv(cuda(x), Wd, normw=cuda(nw), scales=sd))
    cols = np.concatenate([np.sort(r.choice(N - 8, 248, replace=False)), np.arange(N - 8, N)])
    idx = torch.from_numpy(cols).cuda()
    ref = O.gemv(x, host(Wd[idx]), normw=nw, scales=None if sd is None else host(sd[idx]))
    check(name, got[:, cols], ref, 3e-3, 3e-3)


@pytest.mark.parametrize("q", [False, True], ids=["fp16", "int8"])
def test_llama31_8b_lm_head(hi, O, q):
    """C2's lm_head, 4096 -> 128256 with the final RMSNorm fused, at 1 and 8 rows."""
    r = rng(30 + q)
    H = 4096
    Wd, sd = gpu_weights(hi, 30, 128256, H, q)
    nw = (r.random(H) + 0.5).astype(np.float16)
    for M in [1, 8]:
        sampled_lm_head(hi, O, r, Wd, sd, h16(r, M, H), nw, f"C2 lm_head {'int8' if q else 'fp16'} M={M}")


@pytest.mark.parametrize("q", [False, True], ids=["fp16", "int8"])
def test_llama31_8b_o_and_down(hi, O, q):
    """C2's two residual GEMVs at full size, o_proj 4096 -> 4096 and down 14336 -> 4096, called as
    the decode token calls them (epi 1 into the residual stream, the launch shape the host picks for
    N = 4096 at 1 and 8 rows). Every output column is checked against the oracle on the same bytes,
    and row m of the 8-row call must equal the 1-row call of that row bit for bit."""
    r = rng(60 + q)
    H, I = 4096, 14336
    kind = "int8" if q else "fp16"
    for name, K, seed in [("o_proj", H, 60), ("down", I, 61)]:
        Wd, sd = gpu_weights(hi, seed, H, K, q)
        Wh, sh = host(Wd), None if sd is None else host(sd)
        x = h16(r, 8, K)
        if name == "down":  # SwiGLU outputs: small, mostly positive-skewed values
            x = (x * 0.25).astype(np.float16)
        res = h16(r, 8, H)
        ones = []
        for m in range(8):
            out = cuda(res[m:m + 1])
            hi.gemv(cuda(x[m:m + 1]), Wd, out=out, epi=1, scales=sd)
            ones.append(host(out)[0])
            if m == 0:
                ref = O.gemv(x[:1], Wh, out=res[:1].copy(), epi=1, scales=sh)
                check(f"C2 {name} {kind} M=1", host(out), ref, 4e-3, 2e-3)
        out = cuda(res)
        hi.gemv(cuda(x), Wd, out=out, epi=1, scales=sd)
        got = host(out)
        check(f"C2 {name} {kind} M=8", got, O.gemv(x, Wh, out=res.copy(), epi=1, scales=sh), 4e-3, 2e-3)
        for m in range(8):
            assert np.array_equal(bits(got[m]), bits(ones[m])), f"C2 {name} {kind}: row {m} of 8 differs from the 1-row call"


@pytest.mark.parametrize("q", [False, True], ids=["fp16", "int8"])
def test_qwen25_1p5b_shapes(hi, O, q):
    """C4 (Qwen2.5-1.5B) at the batch / verify widths N = 1, 2, 5, 8: fused-norm gate/up + SwiGLU
    1536 -> 2 x 8960, down + residual 8960 -> 1536, fused-norm QKV + bias + RoPE 1536 -> 2048 (12 q
    heads, 2 kv heads, head_dim 128), all checked whole against the oracle, and the 151936-row
    lm_head on sampled columns."""
    r = rng(40 + q)
    H, I, D, Hq, Hkv, S = 1536, 8960, 128, 12, 2, 256
    gu = interleave(h16(r, I, H, sd=0.02), h16(r, I, H, sd=0.02))
    dn = h16(r, H, I, sd=0.02)
    wq = h16(r, (Hq + 2 * Hkv) * D, H, sd=0.02)
    bq = h16(r, (Hq + 2 * Hkv) * D)
    sg = sdn = sq = None
    if q:
        gu, sg = q8(O, gu)
        dn, sdn = q8(O, dn)
        wq, sq = q8(O, wq)
    gud, dnd, wqd = cuda(gu), cuda(dn), cuda(wq)
    sgd, sdnd, sqd = (None, None, None) if not q else (cuda(sg), cuda(sdn), cuda(sq))
    cs = rope_table(S, D)
    nw = (r.random(H) + 0.5).astype(np.float16)
    Wl, sl = gpu_weights(hi, 41, 151936, H, q)
    kind = "int8" if q else "fp16"
    for M in [1, 2, 5, 8]:
        x = h16(r, M, H)
        got = host(hi.gemv(cuda(x), gud, epi=2, normw=cuda(nw), scales=sgd))
        check(f"C4 gate/up {kind} N={M}", got, O.gemv(x, gu, epi=2, normw=nw, scales=sg), 3e-3, 3e-3)
        a = h16(r, M, I)
        res = h16(r, M, H)
        out = cuda(res)
        hi.gemv(cuda(a), dnd, out=out, epi=1, scales=sdnd)
        check(f"C4 down {kind} N={M}", host(out), O.gemv(a, dn, out=res.copy(), epi=1, scales=sdn), 4e-3, 2e-3)
        pos = r.integers(0, S, M).astype(np.int32)
        out_r = np.zeros((M, Hq * D), np.float16)
        kc_r = np.zeros((M, Hkv, S, D), np.float16)
        vc_r = np.zeros_like(kc_r)
        O.gemv_qkv_rope(x, wq, nw, Hq, Hkv, cs, pos, kc_r, vc_r, out_r, bias=bq, scales=sq)
        out = cuda(np.zeros((M, Hq * D), np.float16))
        kc, vc = cuda(np.zeros_like(kc_r)), cuda(np.zeros_like(vc_r))
        hi.gemv_qkv_rope(cuda(x), wqd, cuda(nw), Hq, Hkv, cuda(cs), cuda(pos), kc, vc, out, bias=cuda(bq), scales=sqd)
        check(f"C4 qkv+rope {kind} N={M}: q", host(out), out_r, 2e-2, 2e-3)
        check(f"C4 qkv+rope {kind} N={M}: k cache", host(kc), kc_r, 2e-2, 2e-3)
        check(f"C4 qkv+rope {kind} N={M}: v cache", host(vc), vc_r, 2e-2, 2e-3)
        sampled_lm_head(hi, O, r, Wl, sl, x, nw, f"C4 lm_head {kind} N={M}")


def test_int8_positive_activations_with_outliers(hi, O):
    """int8 weights against all-positive activations with outliers at long K (SwiGLU-like down
    projection inputs, K = 14336, |x| up to 100): the worst case for the cancellation of any offset
    carried through the fp32 sums. Also with the residual epilogue."""
    r = rng(50)
    K, N = 14336, 1024
    W, s = q8(O, h16(r, N, K, sd=0.02))
    for M in [1, 5, 8]:
        x = (np.abs(r.standard_normal((M, K))) * 0.7 + 0.05).astype(np.float16)
        spikes = r.choice(K, 24, replace=False)
        x[:, spikes] = (r.random((M, 24)) * 60 + 40).astype(np.float16)
        got = host(hi.gemv(cuda(x), cuda(W), scales=cuda(s)))
        check(f"int8 positive x K={K} M={M}", got, O.gemv(x, W, scales=s), 2e-3, 2e-3)
        res = h16(r, M, N)
        out = cuda(res)
        hi.gemv(cuda(x), cuda(W), out=out, epi=1, scales=cuda(s))
        check(f"int8 positive x residual M={M}", host(out), O.gemv(x, W, out=res.copy(), epi=1, scales=s), 4e-3, 2e-3)
