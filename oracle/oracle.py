"""numpy front end of the CPU oracle (oracle/hi_oracle.c) -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module, as the
checker. Arrays are numpy: fp16 data as np.float16, int8 weights as np.int8, routing indices as
np.int32, routing weights as np.float32. Each wrapper names the reference code it restates
(file:line under the reference checkout); the C file's header carries the full mapping.
"""
import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")


def build():
    """Compile oracle/hi_oracle.c with its Makefile (gcc, IEEE arithmetic)."""
    subprocess.check_call(["make", "-s", "-C", _HERE])


def _load():
    if not os.path.exists(_LIB_PATH):
        build()
    lib = C.CDLL(_LIB_PATH)
    P, I, I64, F = C.c_void_p, C.c_int, C.c_int64, C.c_float
    sig = {
        "or_f2h_array": ([P, P, I64], None),
        "or_h2f_array": ([P, P, I64], None),
        "or_set_threads": ([I], None),
        "or_get_threads": ([], I),
        "or_quantize_rows": ([P, I64, I64, P, P], I),
        "or_dequantize_rows": ([P, P, I64, I64, P], I),
        "or_interleave_gate_up": ([P, P, I64, I64, P], I),
        "or_deinterleave_gate_up": ([P, I64, I64, P, P], I),
        "or_rmsnorm": ([P, I64, P, I, I, F, P, I64], I),
        "or_silu_mul": ([F, F], C.c_uint16),
        "or_gemv": ([P, I64, P, F, P, P, P, I64, I, I, I, I], I),
        "or_gemv_qkv_rope": ([P, I64, P, F, P, P, P, P, I64, I, I, I, I, I, P, P, P, P, I, I], I),
        "or_gemm": ([P, I64, P, P, P, P, I64, I, I, I, I], I),
        "or_moe_router": ([P, I64, P, I, I, I, I, I, P, P], I),
        "or_moe_experts": ([P, I64, P, P, P, P, I, I, I, I, I, I, F, P, I64], I),
        "or_decode_attn": ([P, I64, P, P, I, P, P, I64, I, I, I, I], I),
        "or_argmax": ([P, I, I, P], I),
        "or_rope_cache": ([P, I64, I, I, I, I, P, P, I, I, P, P, I], I),
        "or_flash_prefill": ([P, I64, P, P, I, P, I64, I, I, I, I, I, P], I),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


lib = _load()


def _p(a):
    return None if a is None else C.c_void_p(a.ctypes.data)


def _c(a, dtype):
    """C-contiguous view/copy with the given dtype (no conversion of values)."""
    a = np.asarray(a)
    assert a.dtype == np.dtype(dtype), f"expected {dtype}, got {a.dtype}"
    return np.ascontiguousarray(a)


def _ok(r, what):
    if r != 0:
        raise ValueError(f"oracle {what}: rejected arguments")


def set_threads(n):
    lib.or_set_threads(int(n))


def get_threads():
    return lib.or_get_threads()


def f2h(f):
    """fp32 -> fp16 (own round-to-nearest-even routine), as np.float16."""
    f = _c(np.asarray(f, np.float32), np.float32)
    h = np.empty(f.shape, np.uint16)
    lib.or_f2h_array(_p(f), _p(h), f.size)
    return h.view(np.float16)


def h2f(h):
    h = _c(np.asarray(h).view(np.uint16), np.uint16)
    f = np.empty(h.shape, np.float32)
    lib.or_h2f_array(_p(h), _p(f), h.size)
    return f


def quantize_rows(w):
    """scripts/export.py:54-68: (q int8 [N, K], s fp16 [N])."""
    w = _c(w, np.float16)
    N, K = w.shape
    q = np.empty((N, K), np.int8)
    s = np.empty(N, np.float16)
    _ok(lib.or_quantize_rows(_p(w), N, K, _p(q), _p(s)), "quantize_rows")
    return q, s


def dequantize_rows(q, s):
    """scripts/export.py:71-73: fp16(q * s)."""
    q, s = _c(q, np.int8), _c(s, np.float16)
    N, K = q.shape
    out = np.empty((N, K), np.float16)
    _ok(lib.or_dequantize_rows(_p(q), _p(s), N, K, _p(out)), "dequantize_rows")
    return out


def interleave_gate_up(g, u):
    """scripts/export.py:97-101 (groups of 16 rows), any row dtype."""
    g, u = np.ascontiguousarray(g), np.ascontiguousarray(u)
    assert g.shape == u.shape and g.dtype == u.dtype
    I = g.shape[0]
    out = np.empty((2 * I,) + g.shape[1:], g.dtype)
    _ok(lib.or_interleave_gate_up(_p(g), _p(u), I, g[0].nbytes, _p(out)), "interleave")
    return out


def deinterleave_gate_up(gu):
    """scripts/ref_engine.py:32-36."""
    gu = np.ascontiguousarray(gu)
    I = gu.shape[0] // 2
    g = np.empty((I,) + gu.shape[1:], gu.dtype)
    u = np.empty_like(g)
    _ok(lib.or_deinterleave_gate_up(_p(gu), I, gu[0].nbytes, _p(g), _p(u)), "deinterleave")
    return g, u


def rmsnorm(x, w, eps=1e-5):
    """src/kernels.cuh:110-125 / HF order."""
    x, w = _c(x, np.float16), _c(w, np.float16)
    M, K = x.shape
    y = np.empty_like(x)
    _ok(lib.or_rmsnorm(_p(x), K, _p(w), M, K, eps, _p(y), K), "rmsnorm")
    return y


def silu_mul(g, u):
    """src/kernels.cuh:100-105 on scalars (fp32 in, fp16 out)."""
    return np.uint16(lib.or_silu_mul(float(g), float(u))).view(np.float16)


def _weights(W, scales):
    if scales is None:
        return _c(W, np.float16), None
    return _c(W, np.int8), _c(scales, np.float16)


def gemv(x, W, out=None, normw=None, eps=1e-5, epi=0, scales=None):
    """out[M, *] (epi) x @ W^T as the reference's gemv_kernel computes it (src/kernels.cuh:164-281)."""
    x = _c(x, np.float16)
    W, scales = _weights(W, scales)
    M, K = x.shape
    N = W.shape[0]
    if out is None:
        out = np.zeros((M, N // 2 if epi == 2 else N), np.float16)
    assert out.flags.c_contiguous and out.dtype == np.float16
    nw = None if normw is None else _c(normw, np.float16)
    _ok(lib.or_gemv(_p(x), K, _p(nw), eps, _p(W), _p(scales), _p(out), out.shape[1], M, N, K, epi), "gemv")
    return out


def gemv_qkv_rope(x, W, normw, Hq, Hkv, cs, pos, kc, vc, out, bias=None, eps=1e-5, scales=None, kv_slot=-1):
    """Fused QKV + bias + RoPE + KV write (src/kernels.cuh:265-278). kc/vc [slots, Hkv, max_seq, D]
    are updated in place; out receives the rotated q heads."""
    x = _c(x, np.float16)
    W, scales = _weights(W, scales)
    M, K = x.shape
    D = kc.shape[-1]
    assert kc.flags.c_contiguous and vc.flags.c_contiguous and out.flags.c_contiguous
    cs = _c(cs, np.float16)
    pos = _c(pos, np.int32)
    nw = None if normw is None else _c(normw, np.float16)
    b = None if bias is None else _c(bias, np.float16)
    _ok(lib.or_gemv_qkv_rope(_p(x), K, _p(nw), eps, _p(W), _p(scales), _p(b), _p(out), out.shape[1], M, K, Hq, Hkv,
                             D, _p(cs), _p(pos), _p(kc), _p(vc), kc.shape[2], kv_slot), "gemv_qkv_rope")
    return out


def gemm(A, W, out=None, epi=0, bias=None, scales=None):
    """C (epi) A @ W^T (src/kernels.cuh:305-506); int8 weights enter as fp16(q * s)."""
    A = _c(A, np.float16)
    W, scales = _weights(W, scales)
    M, K = A.shape
    N = W.shape[0]
    if out is None:
        out = np.zeros((M, N // 2 if epi == 2 else N), np.float16)
    assert out.flags.c_contiguous and out.dtype == np.float16
    b = None if bias is None else _c(bias, np.float16)
    _ok(lib.or_gemm(_p(A), K, _p(W), _p(scales), _p(b), _p(out), out.shape[1], M, N, K, epi), "gemm")
    return out


def moe_router(xn, Wr, k, flags):
    """src/kernels.cuh:2091-2147: (idx [M, k] int32, w [M, k] fp32), descending."""
    xn, Wr = _c(xn, np.float16), _c(Wr, np.float16)
    M, H = xn.shape
    E = Wr.shape[0]
    idx = np.empty((M, k), np.int32)
    w = np.empty((M, k), np.float32)
    _ok(lib.or_moe_router(_p(xn), H, _p(Wr), M, E, H, k, flags, _p(idx), _p(w)), "moe_router")
    return idx, w


def moe_experts(xn, wgu, wdown, idx, w, x, flags, scale=1.0):
    """x += MoE(xn) in place (src/kernels.cuh:2156-2276 numerics)."""
    xn, wgu, wdown = _c(xn, np.float16), _c(wgu, np.float16), _c(wdown, np.float16)
    idx, w = _c(idx, np.int32), _c(w, np.float32)
    assert x.flags.c_contiguous and x.dtype == np.float16
    M, H = xn.shape
    E, I2, _ = wgu.shape
    k = idx.shape[1]
    _ok(lib.or_moe_experts(_p(xn), H, _p(wgu), _p(wdown), _p(idx), _p(w), M, E, k, H, I2 // 2, flags, scale, _p(x), H),
        "moe_experts")
    return x


def decode_attn(q, kc, vc, pos, Hq, Hkv):
    """Decode attention (src/kernels.cuh:1486-1660; tests/test_kernels.py:298-307): q [B, Hq*D];
    kc/vc [B, Hkv, max_seq, D]; query b attends to keys 0..pos[b] of slot b. Returns [B, Hq*D] fp16."""
    q, kc, vc, pos = _c(q, np.float16), _c(kc, np.float16), _c(vc, np.float16), _c(pos, np.int32)
    B, Hkv_, S, D = kc.shape
    assert Hkv_ == Hkv
    out = np.empty((B, Hq * D), np.float16)
    _ok(lib.or_decode_attn(_p(q), q.shape[1], _p(kc), _p(vc), S, _p(pos), _p(out), Hq * D, B, Hq, Hkv, D), "decode_attn")
    return out


def argmax(logits):
    """Greedy token per row (src/kernels.cuh:1883-1931): NaN highest, lowest index on ties, 0 for -inf rows."""
    logits = _c(logits, np.float16)
    B, V = logits.shape
    tok = np.empty(B, np.int32)
    _ok(lib.or_argmax(_p(logits), B, V, _p(tok)), "argmax")
    return tok


def rope_cache(qkv, Hq, Hkv, cs, kc, vc, pos=None, pos_base=0, slot_base=0):
    """RoPE + KV-cache write (src/kernels.cuh:1120-1158), in place like the reference: qkv [M,
    (Hq+2Hkv)*D] gets its q heads rotated; kc/vc [slots, Hkv, max_seq, D] get the rotated k and raw v
    rows; cs [max_seq, D/2, 2] fp16. Returns (qkv, kc, vc)."""
    for a in (qkv, kc, vc):
        assert a.flags.c_contiguous and a.dtype == np.float16
    cs = _c(cs, np.float16)
    M = qkv.shape[0]
    D = kc.shape[-1]
    pp = None if pos is None else _c(pos, np.int32)
    _ok(lib.or_rope_cache(_p(qkv), qkv.shape[1], M, Hq, Hkv, D, _p(cs), None if pp is None else _p(pp), pos_base,
                          slot_base, _p(kc), _p(vc), kc.shape[2]), "rope_cache")
    return qkv, kc, vc


def flash_prefill(q, kc, vc, T, p0, Hq, Hkv, lse=False):
    """Causal prefill attention (src/kernels.cuh:1160-1329; tests/test_kernels.py:288-309): q [T,
    Hq*D] (head h at columns h*D), kc/vc [Hkv, max_seq, D] of one slot, row t at position p0 + t.
    Returns out [T, Hq*D] fp16 (and lse [Hq, T] fp32, log2 domain, when lse=True)."""
    q, kc, vc = _c(q, np.float16), _c(kc, np.float16), _c(vc, np.float16)
    Hkv_, S, D = kc.shape
    assert Hkv_ == Hkv
    out = np.empty((T, Hq * D), np.float16)
    ls = np.empty((Hq, T), np.float32) if lse else None
    _ok(lib.or_flash_prefill(_p(q), q.shape[1], _p(kc), _p(vc), S, _p(out), Hq * D, T, p0, Hq, Hkv, D,
                             None if ls is None else _p(ls)), "flash_prefill")
    return (out, ls) if lse else out
