"""Writer of the reference's weight-file format (scripts/export.py:5-38, writer 222-297) from
arrays already in that layout: the file hi_load (and hipinfer_amd.hipinfer.Engine) reads.

Versions: 2 (dense, fp16), 3 (MoE, 128-byte header), 4 (dense with int8 projections and lm_head,
each an int8 [N, K] tensor followed by its fp16 row scales [N]). Every tensor starts a 256-byte
step after the previous one (zero padding), as the reference writes them; the header is 64 bytes
(128 for version 3). Converting a HF checkpoint (the reference export.py's job: Granite multiplier
folding, RoPE scaling from the HF module) is not this module's: the arrays come in ready.
"""
import struct

import numpy as np

MAGIC = 0x48495046
QTYPE_INT8_ROW = 1


def _f16(a):
    a = np.asarray(a)
    assert a.dtype == np.float16, a.dtype
    return np.ascontiguousarray(a)


def write_weights(path, cfg, W):
    """cfg: vocab, hidden, inter, layers, heads, kv_heads, head_dim, max_pos, eps; optional
    attn_scaling (1.0), window (0), tied (False), moe (None, or (experts, top_k, moe_flags,
    out_scale)). W: inv_freq float32 [head_dim/2]; embed [V, H]; final_norm [H]; lm_head [V, H]
    unless tied; layers: [{attn_norm, wqkv [(heads + 2 kv) D, H], bqkv (optional: all layers or
    none), wo, mlp_norm, then wgu [2I, H] (gate/up interleaved in groups of 16) and wdown [H, I],
    or for MoE router [E, H], ewgu [E, 2I, H], ewdown [E, H, I]}]. A projection is fp16, or an
    (int8 q, fp16 scales) pair, which makes the file version 4."""
    layers = W["layers"]
    assert len(layers) == cfg["layers"]
    proj_keys = ("wqkv", "wo", "wgu", "wdown")
    int8 = isinstance(W.get("lm_head"), tuple) or any(isinstance(l.get(k), tuple) for l in layers for k in proj_keys)
    moe = cfg.get("moe")
    tied = bool(cfg.get("tied", False))
    has_bias = "bqkv" in layers[0] and layers[0]["bqkv"] is not None
    assert all(("bqkv" in l and l["bqkv"] is not None) == has_bias for l in layers), "bqkv in all layers or none"
    if int8:
        assert not moe and not tied, "version 4 (int8) is dense with its own lm_head"
    flags = (1 if tied else 0) | (2 if has_bias else 0) | (4 if moe else 0)
    version = 3 if moe else 4 if int8 else 2
    hdr = struct.pack("<10i2f2i", MAGIC, version, cfg["vocab"], cfg["hidden"], cfg["inter"], cfg["layers"],
                      cfg["heads"], cfg["kv_heads"], cfg["head_dim"], cfg["max_pos"], float(cfg["eps"]),
                      float(cfg.get("attn_scaling", 1.0)), flags, int(cfg.get("window", 0)))
    if moe:
        E, top_k, moe_flags, out_scale = moe
        hdr = hdr.ljust(64, b"\0") + struct.pack("<3if", E, top_k, moe_flags, float(out_scale))
        hdr = hdr.ljust(128, b"\0")
    else:
        if int8:
            hdr += struct.pack("<i", QTYPE_INT8_ROW)
        hdr = hdr.ljust(64, b"\0")

    with open(path, "wb") as f:
        f.write(hdr)

        def put_bytes(b):
            f.write(b)
            f.write(b"\0" * ((-len(b)) % 256))

        def put(a):
            put_bytes(_f16(a).tobytes())

        def put_w(a):
            if isinstance(a, tuple):
                q, s = a
                q = np.ascontiguousarray(np.asarray(q))
                assert q.dtype == np.int8 and np.asarray(s).shape == (q.shape[0],)
                put_bytes(q.tobytes())
                put(s)
            else:
                assert not int8, "an int8 file stores every projection as (q, scales)"
                put(a)

        inv = np.ascontiguousarray(np.asarray(W["inv_freq"], np.float32))
        assert inv.shape == (cfg["head_dim"] // 2,)
        put_bytes(inv.tobytes())
        put(W["embed"])
        put(W["final_norm"])
        if not tied:
            put_w(W["lm_head"])
        for l in layers:
            put(l["attn_norm"])
            put_w(l["wqkv"])
            if has_bias:
                put(l["bqkv"])
            put_w(l["wo"])
            put(l["mlp_norm"])
            if moe:
                put(l["router"])
                put(l["ewgu"])
                put(l["ewdown"])
            else:
                put_w(l["wgu"])
                put_w(l["wdown"])
    return version
