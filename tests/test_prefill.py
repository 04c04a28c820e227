"""GPU parity of the prefill kernels around the GEMM (RoPE + KV-cache write, causal prefill
attention), through the C-ABI, against the CPU oracle on the same seeded inputs.

Mirrors the reference's tests/test_kernels.py test_rope (237-261: D 64/128, GQA 8/3/1, prefill form
at p0 = 100 into slot 2, decode form with per-row positions, exact) and test_flash_prefill
(299-309: D 64/128, GQA groups 8/4/3/1/7, T from 1 to 1024, a prefix p0 of 300 and 1000, tolerance
2e-3 + 1e-2 |ref|). Adds: q read in place from a fused qkv row (ldq > Hq*D), the lse output, and
a padded output stride.
"""
import numpy as np
import pytest

from tests._util import bits, check, cuda, gpu, host, rng

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


def rope_table(S, D, theta=10000.0):
    """[S, D/2, 2] (cos, sin) fp16, built in float32 like the reference's rope_table (test_kernels.py:224-227)."""
    inv = (1.0 / theta ** (np.arange(0, D, 2, dtype=np.int64).astype(np.float32) / D)).astype(np.float32)
    ang = np.arange(S, dtype=np.float32)[:, None] * inv[None, :]
    return np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float16)


@pytest.mark.parametrize("D,Hq,Hkv", [(64, 32, 4), (128, 24, 8), (128, 16, 16)])
def test_rope_cache(hi, O, D, Hq, Hkv):
    r = rng(1000 + D + Hq)
    S, T, p0 = 512, 37, 100
    cs = rope_table(S, D)
    qkv = r.standard_normal((T, (Hq + 2 * Hkv) * D)).astype(np.float16)
    kc = np.zeros((3, Hkv, S, D), np.float16)
    vc = np.zeros_like(kc)
    dq, dk, dv = cuda(qkv), cuda(kc), cuda(vc)
    hi.rope_cache(dq, Hq, Hkv, cuda(cs), dk, dv, pos_base=p0, slot_base=2)
    O.rope_cache(qkv, Hq, Hkv, cs, kc, vc, pos_base=p0, slot_base=2)
    assert np.array_equal(bits(host(dq)), bits(qkv)), "q rotation (prefill form)"
    assert np.array_equal(bits(host(dk)), bits(kc)) and np.array_equal(bits(host(dv)), bits(vc)), "cache (prefill form)"
    # decode form: per-row positions, row b -> slot b
    qkv = r.standard_normal((3, (Hq + 2 * Hkv) * D)).astype(np.float16)
    pos = np.array([5, 400, 0], np.int32)
    dq = cuda(qkv)
    hi.rope_cache(dq, Hq, Hkv, cuda(cs), dk, dv, pos=cuda(pos))
    O.rope_cache(qkv, Hq, Hkv, cs, kc, vc, pos=pos)
    assert np.array_equal(bits(host(dq)), bits(qkv)), "q rotation (decode form)"
    assert np.array_equal(bits(host(dk)), bits(kc)) and np.array_equal(bits(host(dv)), bits(vc)), "cache (decode form)"


@pytest.mark.parametrize("D,Hq,Hkv,pad,offset", [(48, 6, 2, 0, 0), (64, 8, 2, 3, 0), (128, 12, 4, 0, 1),
                                                  (160, 5, 1, 1, 0), (2, 3, 3, 0, 0)],
                         ids=["D48", "odd-ldq", "unaligned-ptr", "D160", "D2"])
def test_rope_cache_any_alignment(hi, O, D, Hq, Hkv, pad, offset):
    """The 2-byte kernel runs whenever the 16-byte one cannot: D % 16 != 0 (D = 48, 160 with 80
    pairs per head so lanes take two, the minimum D = 2), ldq % 8 != 0 (padded rows), or a qkv
    pointer that is not 16-byte aligned. Same bits as the oracle, in both the prefill and the
    decode forms; the row padding stays untouched."""
    r = rng(1300 + D + pad + offset)
    S, T, p0 = 256, 19, 60
    cs = rope_table(S, D)
    W = (Hq + 2 * Hkv) * D + pad
    for form in ["prefill", "decode"]:
        M = T if form == "prefill" else 4
        flat = r.standard_normal(M * W + offset).astype(np.float16)
        qkv = flat[offset:].reshape(M, W).copy()
        kc = np.zeros((M + 3, Hkv, S, D), np.float16)
        vc = np.zeros_like(kc)
        dflat, dk, dv = cuda(flat), cuda(kc), cuda(vc)
        dq = dflat[offset:].view(M, W)
        if form == "prefill":
            hi.rope_cache(dq, Hq, Hkv, cuda(cs), dk, dv, pos_base=p0, slot_base=2)
            O.rope_cache(qkv, Hq, Hkv, cs, kc, vc, pos_base=p0, slot_base=2)
        else:
            pos = np.array([0, S - 1, 7, 100], np.int32)
            hi.rope_cache(dq, Hq, Hkv, cuda(cs), dk, dv, pos=cuda(pos), slot_base=1)
            O.rope_cache(qkv, Hq, Hkv, cs, kc, vc, pos=pos, slot_base=1)
        got = host(dflat)
        assert np.array_equal(bits(got[:offset]), bits(flat[:offset])), "wrote before the rows"
        assert np.array_equal(bits(got[offset:].reshape(M, W)), bits(qkv)), f"q rotation ({form} form)"
        assert np.array_equal(bits(host(dk)), bits(kc)), f"k cache ({form} form)"
        assert np.array_equal(bits(host(dv)), bits(vc)), f"v cache ({form} form)"


FP_HEADS = [(64, 32, 4), (64, 32, 8), (128, 24, 8), (128, 16, 16), (128, 28, 4)]
FP_LENS = [(1, 0), (64, 0), (100, 0), (517, 0), (1024, 0), (70, 300), (33, 1000)]


@pytest.mark.parametrize("D,Hq,Hkv", FP_HEADS, ids=[f"D{d}-G{q // k}" for d, q, k in FP_HEADS])
def test_flash_prefill(hi, O, D, Hq, Hkv):
    r = rng(1100 + D + Hq + Hkv)
    S = 2048
    kc = r.standard_normal((Hkv, S, D)).astype(np.float16)
    vc = r.standard_normal((Hkv, S, D)).astype(np.float16)
    dk, dv = cuda(kc), cuda(vc)
    for T, p0 in FP_LENS:
        q = r.standard_normal((T, Hq * D)).astype(np.float16)
        got = host(hi.flash_prefill(cuda(q), dk, dv, T, p0, Hq, Hkv))
        check(f"flash prefill D={D} G={Hq // Hkv} T={T} p0={p0}", got, O.flash_prefill(q, kc, vc, T, p0, Hq, Hkv),
              2e-3, 1e-2)


def test_flash_prefill_fused_qkv_rows_and_lse(hi, O):
    """q read in place from the rows of a fused qkv buffer (ldq = (Hq + 2 Hkv) D), output into a
    padded buffer (ldo > Hq D, the padding untouched), lse against the oracle's."""
    import torch
    r = rng(1200)
    D, Hq, Hkv, S, T, p0 = 128, 32, 8, 1024, 300, 129
    qkv = r.standard_normal((T, (Hq + 2 * Hkv) * D)).astype(np.float16)
    kc = r.standard_normal((Hkv, S, D)).astype(np.float16)
    vc = r.standard_normal((Hkv, S, D)).astype(np.float16)
    dqkv = cuda(qkv)
    buf = torch.full((T, Hq * D + 64), 7.0, dtype=torch.float16, device="cuda")
    out, lse = hi.flash_prefill_lse(dqkv[:, :Hq * D], cuda(kc), cuda(vc), T, p0, Hq, Hkv, out=buf[:, :Hq * D])
    ref, ref_lse = O.flash_prefill(qkv[:, :Hq * D], kc, vc, T, p0, Hq, Hkv, lse=True)
    check("flash prefill from fused qkv rows", host(out), ref, 2e-3, 1e-2)
    assert (host(buf)[:, Hq * D:] == 7.0).all(), "wrote into the output padding"
    check("flash prefill lse (log2 domain)", host(lse), ref_lse, 1e-4, 1e-5)


@pytest.mark.parametrize("grow", [True, False], ids=["rising", "falling"])
def test_flash_prefill_moving_max(hi, O, grow):
    """Logits that rise (or fall) steeply along the keys: every key share of every tile moves each
    row's running max by far more than the kernel's rescale lag (2^8), so the O rescale and the
    merge of shares with very different maxima run on every tile (with random data a row's max
    settles in its first tiles). Output and lse against the oracle."""
    r = rng(1250 + grow)
    D, Hq, Hkv, S, T, p0 = 128, 16, 8, 1024, 600, 40
    u = np.sign(r.standard_normal(D))  # a fixed direction; q and k lean on it
    pos = np.arange(S, dtype=np.float64)[:, None]
    ramp = 0.03 * (pos if grow else (S - pos))
    kc = (r.standard_normal((Hkv, S, D)) * 0.3 + ramp * u).astype(np.float16)
    vc = r.standard_normal((Hkv, S, D)).astype(np.float16)
    q = (np.tile(u, (T, Hq)) + r.standard_normal((T, Hq * D)) * 0.3).astype(np.float16)
    out, lse = hi.flash_prefill_lse(cuda(q), cuda(kc), cuda(vc), T, p0, Hq, Hkv)
    ref, ref_lse = O.flash_prefill(q, kc, vc, T, p0, Hq, Hkv, lse=True)
    check(f"flash prefill, {'rising' if grow else 'falling'} logits", host(out), ref, 2e-3, 1e-2)
    check(f"flash prefill lse, {'rising' if grow else 'falling'} logits", host(lse), ref_lse, 1e-4, 1e-5)


def test_flash_prefill_rejects_bad_arguments(hi):
    import torch
    q = torch.zeros(4, 3 * 96, dtype=torch.float16, device="cuda")
    kc = torch.zeros(1, 64, 96, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        hi.flash_prefill(q, kc, kc, 4, 0, 3, 1)  # head_dim 96
    q = torch.zeros(4, 2 * 64, dtype=torch.float16, device="cuda")
    kc = torch.zeros(1, 64, 64, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        hi.flash_prefill(q, kc, kc, 4, 61, 2, 1)  # p0 + T past max_seq
    # a cache slot whose head rows pass 2 GiB (32-bit offsets) is refused before anything runs
    out = torch.empty_like(q)
    rc = hi.lib.hi_flash_prefill(hi.ptr(q), q.stride(0), hi.ptr(kc), hi.ptr(kc), 1 << 25, hi.ptr(out), out.stride(0),
                                 4, 0, 2, 1, 64, hi.cur_stream())
    assert rc == -1, rc
