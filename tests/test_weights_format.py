"""CPU checks of the weight-file writer (hipinfer_amd/weights.py) against the reference's format
(scripts/export.py:5-38; the loader's offsets, src/api.cu:1316-1320 `next`: each tensor starts
the 256-byte-rounded size of the previous one later, from byte 64, or 128 for version 3).

The expected header is packed field by field from the format's description, and every tensor is
looked up at the offset that stepping rule gives, then compared with the array written."""
import os
import struct

import numpy as np
import pytest

from tests._util import rng

pytest.importorskip("numpy")


def _model(r, H=64, I=128, L=2, Hq=4, Hkv=2, D=16, V=96, bias=False, moe=None, int8=False, tied=False):
    f = lambda *s: (r.standard_normal(s) * 0.1).astype(np.float16)
    QKV = (Hq + 2 * Hkv) * D

    def proj(n, k):
        w = f(n, k)
        if not int8:
            return w
        s = (np.abs(w.astype(np.float32)).max(1) / 127).astype(np.float16)
        q = np.clip(np.round(w.astype(np.float32) / np.maximum(s.astype(np.float32), 1e-30)[:, None]), -127,
                    127).astype(np.int8)
        return (q, s)

    layers = []
    for _ in range(L):
        ly = {"attn_norm": f(H), "wqkv": proj(QKV, H), "wo": proj(H, Hq * D), "mlp_norm": f(H)}
        if bias:
            ly["bqkv"] = f(QKV)
        if moe:
            E = moe[0]
            ly.update(router=f(E, H), ewgu=f(E, 2 * I, H), ewdown=f(E, H, I))
        else:
            ly.update(wgu=proj(2 * I, H), wdown=proj(H, I))
        layers.append(ly)
    W = {"inv_freq": (1.0 / 10000.0 ** (np.arange(0, D, 2) / D)).astype(np.float32), "embed": f(V, H),
         "final_norm": f(H), "layers": layers}
    if not tied:
        W["lm_head"] = proj(V, H)
    cfg = dict(vocab=V, hidden=H, inter=I, layers=L, heads=Hq, kv_heads=Hkv, head_dim=D, max_pos=4096, eps=1e-5,
               attn_scaling=1.0, window=0, tied=tied, moe=moe)
    return cfg, W


def _expected_tensors(cfg, W):
    """(array, bytes) in file order, as the reference's writer emits them."""
    out = [W["inv_freq"], W["embed"], W["final_norm"]]

    def proj(a):
        return list(a) if isinstance(a, tuple) else [a]
    if not cfg.get("tied"):
        out += proj(W["lm_head"])
    for l in W["layers"]:
        out += [l["attn_norm"]] + proj(l["wqkv"]) + ([l["bqkv"]] if "bqkv" in l else []) + proj(l["wo"]) + \
            [l["mlp_norm"]]
        out += [l["router"], l["ewgu"], l["ewdown"]] if cfg.get("moe") else proj(l["wgu"]) + proj(l["wdown"])
    return out


@pytest.mark.parametrize("kind", ["dense", "bias_tied", "int8", "moe"])
def test_writer_matches_the_format(tmp_path, kind):
    from hipinfer_amd.weights import MAGIC, write_weights
    r = rng(60)
    kw = dict(dense={}, bias_tied=dict(bias=True, tied=True), int8=dict(int8=True),
              moe=dict(moe=(4, 2, 3, 0.5)))[kind]
    cfg, W = _model(r, **kw)
    path = os.path.join(tmp_path, "m.bin")
    ver = write_weights(path, cfg, W)
    blob = open(path, "rb").read()
    want_ver = {"dense": 2, "bias_tied": 2, "int8": 4, "moe": 3}[kind]
    assert ver == want_ver
    # header: int32 magic, version, vocab, hidden, inter, layers, heads, kv_heads, head_dim, max_pos,
    # float eps, attention_scaling, int32 flags, sliding_window; v4: qtype at 56; v3: MoE at 64
    h = struct.unpack_from("<10i2f2i", blob, 0)
    assert h[:10] == (MAGIC, want_ver, cfg["vocab"], cfg["hidden"], cfg["inter"], cfg["layers"], cfg["heads"],
                      cfg["kv_heads"], cfg["head_dim"], cfg["max_pos"])
    assert abs(h[10] - 1e-5) < 1e-12 and h[11] == 1.0 and h[13] == 0
    flags = (1 if kind == "bias_tied" else 0) | (2 if kind == "bias_tied" else 0) | (4 if kind == "moe" else 0)
    assert h[12] == flags
    if kind == "int8":
        assert struct.unpack_from("<i", blob, 56)[0] == 1
    if kind == "moe":
        assert struct.unpack_from("<3if", blob, 64) == (4, 2, 3, 0.5)
    base = 128 if kind == "moe" else 64
    pad = [(60, 64)] if kind == "int8" else [(56, 64), (80, 128)] if kind == "moe" else [(56, 64)]
    for lo, hi in pad:
        assert blob[lo:hi] == b"\0" * (hi - lo), ("header padding", lo, hi)
    off = base
    for a in _expected_tensors(cfg, W):
        b = np.ascontiguousarray(a).tobytes()
        assert blob[off:off + len(b)] == b, (kind, off)
        assert blob[off + len(b):off + (len(b) + 255) // 256 * 256].strip(b"\0") == b"", "padding must be zeros"
        off += (len(b) + 255) // 256 * 256
    assert len(blob) == off, "no bytes after the last tensor's padding"
