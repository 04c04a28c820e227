"""GPU parity of the decode-step kernels around the GEMVs (decode attention, greedy argmax,
embedding gather), through the C-ABI, against the CPU oracle on the same seeded inputs.

Mirrors the reference's tests/test_kernels.py test_decode_attn (335-345: D 64/128, GQA groups 1..8,
context lengths 1..4000 in one batch, max_seq 4096, tolerance 2e-3 + 1e-2 |ref|),
test_decode_work_reuse (348-355: one zeroed work buffer shared by launches of B = 8, 1, 4, 16, 2)
and test_argmax (208-221). Adds: a captured graph replayed while the context grows (the split
count is derived on the device), and the exact embedding gather.
"""
import numpy as np
import pytest

from tests._util import check, cuda, gpu, host, rng

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


def attn_case(hi, O, lens, Hq, Hkv, D, S, seed, work=None):
    r = rng(seed)
    B = len(lens)
    q = (r.standard_normal((B, Hq * D))).astype(np.float16)
    kc = (r.standard_normal((B, Hkv, S, D))).astype(np.float16)
    vc = (r.standard_normal((B, Hkv, S, D))).astype(np.float16)
    pos = np.array([l - 1 for l in lens], np.int32)
    got = host(hi.decode_attn(cuda(q), cuda(kc), cuda(vc), cuda(pos), Hq, Hkv, work=work))
    ref = O.decode_attn(q, kc, vc, pos, Hq, Hkv)
    return got, ref


CASES = [[1], [37], [4000], [1, 300, 1024, 2049], list(range(5, 4000, 250))]
GROUPS = [(64, 8), (64, 4), (64, 1), (128, 4), (128, 3), (128, 1), (128, 7), (64, 7), (128, 8), (64, 2), (128, 6),
          (64, 5)]


@pytest.mark.parametrize("D,G", GROUPS, ids=[f"D{d}-G{g}" for d, g in GROUPS])
def test_decode_attn(hi, O, D, G):
    Hkv = 4 if G != 1 else 16
    for i, lens in enumerate(CASES):
        got, ref = attn_case(hi, O, lens, Hkv * G, Hkv, D, 4096, 500 + 10 * D + G + i)
        check(f"decode attn D={D} G={G} lens={lens if len(lens) <= 4 else f'{lens[0]}..{lens[-1]}'}", got, ref,
              2e-3, 1e-2)


def test_decode_attn_batch64(hi, O):
    """The batched decode step's shape (Llama-3.1-8B: Hkv 8, G 4, D 128) at 64 sequences and about
    1024 positions: one split per (sequence, kv head), so each wave runs four tiles in turn with the
    next tile's K and V in flight during the current one; ragged lengths end tiles part-way."""
    lens = [1024 - 13 * i for i in range(64)]
    got, ref = attn_case(hi, O, lens, 32, 8, 128, 1040, 650)
    check("decode attn B=64 lens=1024..205", got, ref, 2e-3, 1e-2)


def test_decode_work_reuse(hi, O):
    """One zeroed work buffer for launches of decreasing and increasing batch: the split counters
    must be left zeroed and never land in a larger launch's partials. One kv head per sequence
    means many splits per launch."""
    import torch
    D, Hkv, G = 128, 1, 4
    work = torch.zeros(hi.lib.hi_decode_work_bytes(16, Hkv * G, Hkv, D), dtype=torch.uint8, device="cuda")
    for B in [8, 1, 4, 16, 2]:
        got, ref = attn_case(hi, O, [2000 - 97 * b for b in range(B)], Hkv * G, Hkv, D, 2048, 600 + B, work=work)
        check(f"decode attn shared work B={B}", got, ref, 2e-3, 1e-2)
    assert int(work[:4096 * 4].view(torch.int32).abs().sum()) == 0, "split counters not left zeroed"


def test_decode_attn_graph_replay_growing_context(hi, O):
    """A captured launch stays valid as pos advances (the kernel reads pos on the device and picks
    its split count from it); every replay matches the oracle."""
    import torch
    r = rng(700)
    B, Hkv, G, D, S = 3, 8, 4, 128, 4096
    Hq = Hkv * G
    q = r.standard_normal((B, Hq * D)).astype(np.float16)
    kc = r.standard_normal((B, Hkv, S, D)).astype(np.float16)
    vc = r.standard_normal((B, Hkv, S, D)).astype(np.float16)
    qd, kd, vd = cuda(q), cuda(kc), cuda(vc)
    pos = torch.zeros(B, dtype=torch.int32, device="cuda")
    out = torch.empty(B, Hq * D, dtype=torch.float16, device="cuda")
    work = torch.zeros(hi.lib.hi_decode_work_bytes(B, Hq, Hkv, D), dtype=torch.uint8, device="cuda")
    hi.decode_attn(qd, kd, vd, pos, Hq, Hkv, out=out, work=work)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        hi.decode_attn(qd, kd, vd, pos, Hq, Hkv, out=out, work=work)
    for p in [[0, 5, 63], [64, 255, 256], [1000, 2047, 4095], [3, 700, 1500]]:
        pn = np.array(p, np.int32)
        pos.copy_(torch.from_numpy(pn))
        g.replay()
        torch.cuda.synchronize()
        check(f"decode attn graph replay pos={p}", host(out), O.decode_attn(q, kc, vc, pn, Hq, Hkv), 2e-3, 1e-2)


def test_argmax(hi, O):
    """The reference's cases (ties to the lowest index, NaN wins, all -inf and all NaN rows give 0,
    +inf), exact against the oracle, plus vocabulary-sized random rows and an odd V whose rows are
    not 16-byte aligned."""
    import torch
    r = rng(710)
    V = 32000
    lg = r.standard_normal((6, V)).astype(np.float16)
    lg[1, 100] = lg[1, 31999] = 20.0
    lg[2, 5000] = np.nan
    lg[2, 7] = np.nan
    lg[3] = -np.inf
    lg[4] = np.nan
    lg[5, 31999] = np.inf
    got = host(hi.argmax(cuda(lg)))
    assert np.array_equal(got, O.argmax(lg)), got
    for V in [128256, 151936, 32001, 7]:
        lg = r.standard_normal((5, V)).astype(np.float16)
        lg[0, V // 3] = lg[0, V - 1] = 30.0  # a tie far apart
        got = host(hi.argmax(cuda(lg)))
        assert np.array_equal(got, O.argmax(lg)), (V, got)
    assert host(hi.argmax(torch.zeros(0, 10, dtype=torch.float16, device="cuda"))).shape == (0,)


def test_embed(hi):
    r = rng(720)
    V, H = 1000, 2048
    table = r.standard_normal((V, H)).astype(np.float16)
    tok = np.array([0, 999, 17, 17, 500], np.int32)
    got = host(hi.embed(cuda(tok), cuda(table)))
    assert np.array_equal(got, table[tok])
