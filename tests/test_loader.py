"""GPU parity of the engine entry points (hi_load, hi_prefill, hi_decode, hi_history, hi_logits,
hi_rewind, hi_set_state; the reference's load_shard / prefill / decode_step / accessors,
src/api.cu:1235-1546, 1807-2178) through hipinfer_amd.hipinfer.Engine, the mirror of the
reference's Python Engine (scripts/hipinfer.py:334-500), on small random models written in the
reference's weight-file format: fp16 with a QKV bias, tied embeddings, int8 projections (version
4), and MoE (version 3).

Each model is checked against the same computation chained from the CPU oracle: the prefill's
last-position logits and greedy token (prompt in three chunks), then decode steps one at a time
(the engine is put back on the oracle's token with hi_rewind, so a near-tie cannot fork the two),
then two slots decoding together. Engine.generate with and without graphs must agree token for
token. A wrong weight offset, a mis-built RoPE table or a missing bias shows up as a logits
mismatch at the first comparison.
"""
import os

import numpy as np
import pytest

from tests._util import check, gpu, host, interleave, rng

pytestmark = gpu

C = dict(H=512, Hq=8, Hkv=2, D=64, I=1024, V=2048, L=2, eps=1e-5, E=8, k=2, EI=256)


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


def make_model(O, r, kind):
    """(file cfg, file arrays, oracle view {embed, lm, nf, layers}) for kind in dense_bias, tied, int8, moe."""
    H, Hq, Hkv, D, I, V, L = (C[k] for k in ("H", "Hq", "Hkv", "D", "I", "V", "L"))
    w = lambda n, k, sd=0.05: (r.standard_normal((n, k)) * sd).astype(np.float16)
    nrm = lambda: (r.random(H) + 0.5).astype(np.float16)
    q8 = kind == "int8"
    pj = lambda a: O.quantize_rows(a) if q8 else a
    layers, olayers = [], []
    for _ in range(L):
        ly = {"attn_norm": nrm(), "wqkv": pj(w((Hq + 2 * Hkv) * D, H)), "wo": pj(w(H, Hq * D)), "mlp_norm": nrm()}
        if kind == "dense_bias":
            ly["bqkv"] = (r.standard_normal((Hq + 2 * Hkv) * D) * 0.1).astype(np.float16)
        if kind == "moe":
            E, EI = C["E"], C["EI"]
            ly["router"] = w(E, H, 0.5)
            ly["ewgu"] = np.stack([interleave(w(EI, H), w(EI, H)) for _ in range(E)])
            ly["ewdown"] = np.stack([w(H, EI, 0.03) for _ in range(E)])
        else:
            ly["wgu"] = pj(interleave(w(I, H), w(I, H)))
            ly["wdown"] = pj(w(H, I, 0.03))
        layers.append(ly)
        olayers.append(ly)
    inv = (1.0 / (500000.0 ** (np.arange(0, D, 2, dtype=np.int64).astype(np.float32) / D))).astype(np.float32)
    tied = kind == "tied"
    # a tied head is the embedding: give it the scale the untied heads have
    embed = (r.standard_normal((V, H)) * (0.05 if tied else 1.0)).astype(np.float16)
    W = {"inv_freq": inv, "embed": embed, "final_norm": nrm(), "layers": layers}
    if not tied:
        W["lm_head"] = pj(w(V, H))
    cfg = dict(vocab=V, hidden=H, inter=C["EI"] if kind == "moe" else I, layers=L, heads=Hq, kv_heads=Hkv, head_dim=D,
               max_pos=8192, eps=C["eps"], attn_scaling=1.0, window=0, tied=tied,
               moe=(C["E"], C["k"], 1, 0.75) if kind == "moe" else None)
    ov = {"embed": embed, "lm": embed if tied else W["lm_head"], "nf": W["final_norm"], "layers": olayers, "cfg": cfg}
    return cfg, W, ov


def rope_table(inv, S, scaling=1.0):
    """The engine's table: fp32 angle p * inv_freq, cos / sin of it (double) to fp32, x scaling, fp16."""
    a = np.arange(S, dtype=np.float32)[:, None] * inv[None, :]
    c = np.cos(a.astype(np.float64)).astype(np.float32) * np.float32(scaling)
    s = np.sin(a.astype(np.float64)).astype(np.float32) * np.float32(scaling)
    return np.stack([c, s], -1).astype(np.float16)


def _ws(a):
    return (a[0], a[1]) if isinstance(a, tuple) else (a, None)


def o_mlp(O, ov, ly, x):
    eps, cfg = C["eps"], ov["cfg"]
    xn = O.rmsnorm(x, ly["mlp_norm"], eps)
    if cfg["moe"]:
        E, k, flags, scale = cfg["moe"]
        idx, wts = O.moe_router(xn, ly["router"], k, flags)
        return O.moe_experts(xn, ly["ewgu"], ly["ewdown"], idx, wts, x, flags, scale)
    Wg, sg = _ws(ly["wgu"])
    act = O.gemm(xn, Wg, epi=2, scales=sg)
    Wd, sd = _ws(ly["wdown"])
    return O.gemm(act, Wd, out=x, epi=1, scales=sd)


def o_prefill(O, ov, toks, p0, slot, kc, vc, cs):
    Hq, Hkv, D, eps = C["Hq"], C["Hkv"], C["D"], C["eps"]
    T = len(toks)
    x = ov["embed"][np.asarray(toks)].copy()
    for l, ly in enumerate(ov["layers"]):
        xn = O.rmsnorm(x, ly["attn_norm"], eps)
        Wq, sq = _ws(ly["wqkv"])
        qkv = O.gemm(xn, Wq, bias=ly.get("bqkv"), scales=sq)
        O.rope_cache(qkv, Hq, Hkv, cs, kc[l], vc[l], pos_base=p0, slot_base=slot)
        att = O.flash_prefill(np.ascontiguousarray(qkv[:, :Hq * D]), kc[l][slot], vc[l][slot], T, p0, Hq, Hkv)
        Wo, so = _ws(ly["wo"])
        x = O.gemm(att, Wo, out=x, epi=1, scales=so)
        x = o_mlp(O, ov, ly, x)
    Wl, sl = _ws(ov["lm"])
    lg = O.gemv(x[-1:], Wl, normw=ov["nf"], eps=eps, scales=sl)
    return lg, int(O.argmax(lg)[0])


def o_decode(O, ov, tok, pos, kc, vc, cs):
    """B sequences (row b = slot b) through the GEMV-path step."""
    Hq, Hkv, D, eps = C["Hq"], C["Hkv"], C["D"], C["eps"]
    B = len(tok)
    x = ov["embed"][np.asarray(tok)].copy()
    for l, ly in enumerate(ov["layers"]):
        q = np.zeros((B, Hq * D), np.float16)
        Wq, sq = _ws(ly["wqkv"])
        O.gemv_qkv_rope(x, Wq, ly["attn_norm"], Hq, Hkv, cs, np.asarray(pos, np.int32), kc[l], vc[l], q,
                        bias=ly.get("bqkv"), eps=eps, scales=sq)
        att = O.decode_attn(q, kc[l][:B], vc[l][:B], np.asarray(pos, np.int32), Hq, Hkv)
        Wo, so = _ws(ly["wo"])
        x = O.gemv(att, Wo, out=x, epi=1, scales=so)
        if ov["cfg"]["moe"]:
            x = o_mlp(O, ov, ly, x)
        else:
            Wg, sg = _ws(ly["wgu"])
            act = O.gemv(x, Wg, epi=2, normw=ly["mlp_norm"], eps=eps, scales=sg)
            Wd, sd = _ws(ly["wdown"])
            x = O.gemv(act, Wd, out=x, epi=1, scales=sd)
    Wl, sl = _ws(ov["lm"])
    lg = O.gemv(x, Wl, normw=ov["nf"], eps=eps, scales=sl)
    return lg, O.argmax(lg)


def clear(lg, tol=5e-2):
    top2 = np.sort(lg.astype(np.float64), axis=-1)[..., -2:]
    return (top2[..., 1] - top2[..., 0]) > tol


@pytest.mark.parametrize("kind", ["dense_bias", "tied", "int8", "moe"])
def test_engine_from_weight_file_vs_oracle_chain(hi, O, tmp_path, kind, monkeypatch):
    from hipinfer_amd.weights import write_weights
    r = rng(1500 + ["dense_bias", "tied", "int8", "moe"].index(kind))
    cfg, W, ov = make_model(O, r, kind)
    path = os.path.join(tmp_path, f"{kind}.bin")
    write_weights(path, cfg, W)
    S = 96
    e = hi.Engine(path, max_batch=2, max_seq=S, max_prefill=16)
    try:
        assert (e.vocab, e.hidden, e.layers, e.heads, e.kv_heads, e.head_dim) == (C["V"], C["H"], C["L"], C["Hq"],
                                                                                 C["Hkv"], C["D"])
        assert e.quant == (1 if kind == "int8" else 0) and e.tied == (kind == "tied")
        assert e.qkv_bias == (kind == "dense_bias") and e.n_experts == (C["E"] if kind == "moe" else 0)
        cs = rope_table(W["inv_freq"], S)
        kc = [np.zeros((2, C["Hkv"], S, C["D"]), np.float16) for _ in range(C["L"])]
        vc = [np.zeros_like(k) for k in kc]
        tol = 3e-2
        # ---- prefill slot 0 (three chunks of at most 16 rows)
        A = r.integers(0, C["V"], 37).tolist()
        tok = e.prefill(0, A)
        ref_lg, ref_tok = o_prefill(O, ov, A, 0, 0, kc, vc, cs)
        check(f"{kind} prefill logits", host(e.logits(1)), ref_lg, tol, tol)
        if clear(ref_lg)[0]:
            assert tok == ref_tok
        assert e.history(0, 37, 1) == [tok], "the prefill's token is recorded at position T"
        # ---- decode slot 0, one step at a time, each from the oracle's token
        pos, t = 37, ref_tok
        for step in range(3):
            e.rewind(0, pos, t)
            e.decode(1, 1)
            ref_lg, ref_t = o_decode(O, ov, [t], [pos], kc, vc, cs)
            check(f"{kind} decode step {step} logits", host(e.logits(1)), ref_lg, tol, tol)
            got = e.history(0, pos + 1, 1)[0]
            if clear(ref_lg)[0]:
                assert got == int(ref_t[0]), (kind, step)
            pos, t = pos + 1, int(ref_t[0])
        # ---- a second slot, then both slots in one batch
        Bp = r.integers(0, C["V"], 10).tolist()
        e.prefill(1, Bp)
        ref_lg1, ref_tok1 = o_prefill(O, ov, Bp, 0, 1, kc, vc, cs)
        e.set_state([t, ref_tok1], [pos, 10])
        # the two-slot step's gate/up, down and lm_head: the shape rule's choice (dense_bias, moe), or all
        # three forced onto the GEMM path (tied, int8)
        if kind in ("tied", "int8"):
            monkeypatch.setenv("HIPINFER_SMALL_GEMM", "7")
        e.decode(2, 1)
        ref_lg, ref_t = o_decode(O, ov, [t, ref_tok1], [pos, 10], kc, vc, cs)
        check(f"{kind} two-slot decode logits", host(e.logits(2)), ref_lg, tol, tol)
        # ---- argument checks
        with pytest.raises(ValueError):
            e.prefill(0, [C["V"]])  # token outside the vocabulary
        with pytest.raises(ValueError):
            e.decode(3, 1)  # B above max_batch
        with pytest.raises(ValueError):
            e.prefill(2, [1])  # slot outside max_batch
    finally:
        e.close()


def test_generate_graph_and_eager_agree(hi, O, tmp_path):
    """Engine.generate (prefill + hi_decode + hi_history) gives the same tokens with the decode step
    captured as a hipGraph and run eagerly; the first comes from the prefill."""
    from hipinfer_amd.weights import write_weights
    r = rng(1600)
    cfg, W, _ = make_model(O, r, "dense_bias")
    path = os.path.join(tmp_path, "m.bin")
    write_weights(path, cfg, W)
    prompt = r.integers(0, C["V"], 21).tolist()
    a = hi.Engine(path, max_batch=1, max_seq=64, max_prefill=32)
    b = hi.Engine(path, max_batch=1, max_seq=64, max_prefill=32)
    try:
        ta = a.generate(prompt, 12, graph=True)
        tb = b.generate(prompt, 12, graph=False)
        assert ta == tb and len(ta) == 12
        assert ta[0] == a.prefill(0, prompt), "prefill is repeatable"
        assert a.generate(prompt, 12, graph=True) == ta, "the captured graph replays the same tokens"
    finally:
        a.close()
        b.close()


@pytest.mark.parametrize("kind", ["dense_bias", "int8"])
def test_verify_is_bit_identical_to_greedy_decode(hi, O, tmp_path, kind):
    """hi_verify (the reference's speculative verification, api.cu:2018-2108): R draft tokens in one
    pass give, row for row, the logits and greedy token that plain batch-of-one decode steps give
    when fed the same tokens at the same positions -- bit for bit -- eagerly and as a graph replay;
    the slot's state is left alone, and hi_rewind then continues decoding from an accepted prefix."""
    from hipinfer_amd.weights import write_weights
    r = rng(1700 + (kind == "int8"))
    cfg, W, _ = make_model(O, r, kind)
    path = os.path.join(tmp_path, f"{kind}.bin")
    write_weights(path, cfg, W)
    prompt = r.integers(0, C["V"], 23).tolist()
    a = hi.Engine(path, max_batch=2, max_seq=80, max_prefill=32)
    b = hi.Engine(path, max_batch=2, max_seq=80, max_prefill=32)
    try:
        assert a.MAX_VERIFY == 16  # the reference's kGemvMaxRows (api.cu:156, 2066)
        p0 = len(prompt)
        first = a.prefill(0, prompt)
        assert b.prefill(0, prompt) == first
        # 9..16 rows run the fused-norm projections as two launches; every row stays bit-identical
        for R, graph in [(1, False), (5, False), (8, True), (8, True), (3, True), (9, False), (12, True), (16, True),
                         (16, True), (16, False)]:
            draft = [first] + r.integers(0, C["V"], R - 1).tolist()
            toks, lg = a.verify(0, draft, p0, graph=graph, logits=True)
            lg = host(lg)
            for i in range(R):
                b.rewind(0, p0 + i, draft[i])
                b.decode(1, 1)
                ref = host(b.logits(1))[0]
                assert np.array_equal(lg[i].view(np.uint16), ref.view(np.uint16)), (kind, R, graph, i)
                assert toks[i] == b.history(0, p0 + i + 1, 1)[0], (kind, R, graph, i)
        # the slot's own state was left alone: decoding from it continues from the prefill's token
        a.rewind(0, p0, first)
        b.rewind(0, p0, first)
        a.decode(1, 4)
        b.decode(1, 4, graph=False)
        assert a.history(0, p0 + 1, 4) == b.history(0, p0 + 1, 4)
        with pytest.raises(ValueError):
            a.verify(0, [1] * 17, p0)  # more rows than hi_verify_max_rows
    finally:
        a.close()
        b.close()


@pytest.mark.parametrize("E,k", [(257, 2), (32, 17)], ids=["experts_over_256", "top_k_over_16"])
def test_load_rejects_moe_shapes_the_kernels_do_not_take(hi, tmp_path, capfd, E, k):
    """A version-3 header whose expert count or top-k exceeds what the MoE kernels take (256
    experts, top-16) is refused by hi_load, before any weight is read, instead of failing at the
    first MoE call."""
    hdr = np.zeros(32, np.int32)
    hdr[:10] = [0x48495046, 3, 2048, 512, 256, 2, 8, 2, 64, 8192]  # magic, version, vocab, hidden, ...
    hdr[10:12] = np.array([1e-5, 1.0], np.float32).view(np.int32)
    hdr[12] = 4  # MoE
    hdr[16:19] = [E, k, 1]
    hdr[19] = np.array([0.75], np.float32).view(np.int32)[0]
    path = tmp_path / "moe_header_only.bin"
    path.write_bytes(hdr.tobytes())
    with pytest.raises(RuntimeError, match="loading"):
        hi.Engine(str(path), max_batch=1, max_seq=64, max_prefill=64)
    assert "unsupported MoE shape" in capfd.readouterr().err
