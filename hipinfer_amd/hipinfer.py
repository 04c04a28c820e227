"""ctypes host for libhipinfer.so: the matmul hot path of hipinfer on torch tensors.

Mirrors the kernel-level functions of the reference's scripts/hipinfer.py (gemv, gemv_qkv_rope,
gemm, moe_router, moe_experts, rmsnorm, decode_attn; hipinfer.py:101-190, 288-306) with the same names,
arguments and defaults, over the same hi_* C symbols, plus the int8 quantiser of
scripts/export.py:54-101 (quantize_rows, dequantize_rows, interleave_gate_up) running on the GPU.
torch is only the container for device memory and the current stream.

Errors: a launcher that rejects its arguments returns a negative code (the reason is printed on
stderr); these wrappers raise ValueError then. There is no CPU fallback: without the built library
or a GPU every call fails.
"""
import ctypes as C
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = os.environ.get("HIPINFER_LIB", os.path.join(_HERE, "libhipinfer.so"))
if not os.path.exists(_LIB):
    raise ImportError(f"hipinfer_amd: {_LIB} is not built; run `python -m hipinfer_amd.build`")
lib = C.CDLL(os.path.abspath(_LIB))

P, I, F, LL = C.c_void_p, C.c_int, C.c_float, C.c_longlong
_SIGS = {
    "hi_rmsnorm": [P, P, P, I, I, F, P],
    "hi_gemv": [P, I, P, F, P, P, I, I, I, I, I, P],
    "hi_gemv_w8": [P, I, P, F, P, P, P, I, I, I, I, I, P],
    "hi_gemv_qkv_rope": [P, I, P, F, P, P, P, I, I, I, I, I, I, P, P, P, P, I, P],
    "hi_gemv_qkv_rope_w8": [P, I, P, F, P, P, P, P, I, I, I, I, I, I, P, P, P, P, I, P],
    "hi_quantize_rows": [P, LL, I, P, P, P],
    "hi_dequantize_rows": [P, P, LL, I, P, P],
    "hi_device_cus": [],
}
_OPTIONAL = {
    "hi_gemm": [P, I, P, P, P, I, I, I, I, I, P],
    "hi_gemm_w8": [P, I, P, P, P, P, I, I, I, I, I, P],
    "hi_gemm_force_config": [I],
    "hi_gemm_force_splits": [I],
    "hi_gemm_num_configs": [],
    "hi_gemm_config_desc": [I, C.c_char_p, I],
    "hi_moe_router": [P, I, P, I, I, I, I, I, P, P, P],
    "hi_moe_work_bytes": [I, I, I, I, I],
    "hi_moe_experts": [P, I, P, P, P, P, I, I, I, I, I, I, F, P, I, I, P, P],
    "hi_moe_route_experts": [P, I, P, P, P, I, I, I, I, I, I, F, P, I, P, P, P, P],
    "hi_decode_work_bytes": [I, I, I, I],
    "hi_decode_attn": [P, I, P, P, I, P, P, I, I, I, I, I, P, P],
    "hi_argmax": [P, I, I, P, P],
    "hi_embed": [P, P, I, I, P, I, I, P],
    "hi_rope_cache": [P, I, I, I, I, I, P, P, I, I, P, P, I, P],
    "hi_flash_prefill": [P, I, P, P, I, P, I, I, I, I, I, I, P],
    "hi_flash_prefill_lse": [P, I, P, P, I, P, I, I, I, I, I, I, P, P],
    # engine (one GPU)
    "hi_load": [C.c_char_p, I, I, I],
    "hi_load_tp": [C.c_char_p, I, I, I, I, P],
    "hi_free": [P],
    "hi_config": [P, P],
    "hi_moe_config": [P, P],
    "hi_weight_bytes": [P],
    "hi_weight_quant": [P],
    "hi_prefill": [P, I, P, I, I],
    "hi_prefill_logits": [P, I, P, I, I, P],
    "hi_decode": [P, I, I, I],
    "hi_history": [P, I, I, I, P],
    "hi_logits": [P, I, P],
    "hi_set_state": [P, I, P, P],
    "hi_rewind": [P, I, I, I],
    "hi_sync": [P],
    "hi_stream": [P],
    "hi_verify_max_rows": [],
    "hi_verify": [P, I, P, I, I, P, P, I],
}
for _name, _args in list(_SIGS.items()) + [(n, a) for n, a in _OPTIONAL.items() if hasattr(lib, n)]:
    _fn = getattr(lib, _name)
    _fn.argtypes = _args
    _fn.restype = I
for _name, _rt in [("hi_moe_work_bytes", C.c_size_t), ("hi_decode_work_bytes", C.c_size_t),
                   ("hi_weight_bytes", C.c_size_t), ("hi_load", P), ("hi_load_tp", P), ("hi_decode", F),
                   ("hi_stream", P), ("hi_free", None), ("hi_config", None), ("hi_moe_config", None), ("hi_sync", None)]:
    if hasattr(lib, _name):
        getattr(lib, _name).restype = _rt
MOE_NORM_TOPK, MOE_FP16_WEIGHTS = 1, 2  # moe_flags bits (reference scripts/hipinfer.py:67)


def _s():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _p(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def _ok(r, what):
    if r != 0:
        raise ValueError(f"hipinfer_amd {what}: rejected (code {r}; reason on stderr)")


def _dev(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("hipinfer_amd: tensors must live on the GPU")


# W [N, K]: fp16, or int8 with `scales` [N] fp16 (one per output row: W ~ W_int8 * scales[:, None]).
def _w8(W, scales):
    if scales is None:
        assert W.dtype == torch.float16
        return False
    assert W.dtype == torch.int8 and scales.dtype == torch.float16 and scales.shape == (W.shape[0],)
    return True


def rmsnorm(x, w, eps=1e-5, out=None):
    """y = w * fp16(x * rsqrt(mean(x^2) + eps)) per row of x [M, H] (contiguous rows)."""
    y = torch.empty_like(x) if out is None else out
    _dev(x, w, y)
    if not (x.is_contiguous() and y.is_contiguous()):
        raise ValueError("hipinfer_amd: rmsnorm rows must be contiguous")
    _ok(lib.hi_rmsnorm(_p(x), _p(w), _p(y), x.shape[0], x.shape[1], eps, _s()), "rmsnorm")
    return y


def gemv(x, W, out=None, normw=None, eps=1e-5, epi=0, scales=None):
    """out[M, *] (epi) x[M, K] @ W[N, K]^T for small M; epi 0 store, 1 residual (out += y),
    2 SwiGLU over gate/up rows interleaved in groups of 16 (out is N/2 wide)."""
    M, K = x.shape
    N = W.shape[0]
    if out is None:
        out = torch.empty(M, N // 2 if epi == 2 else N, dtype=x.dtype, device=x.device)
    _dev(x, W, out, normw, scales)
    if _w8(W, scales):
        r = lib.hi_gemv_w8(_p(x), x.stride(0), _p(normw), eps, _p(W), _p(scales), _p(out), out.stride(0), M, N, K, epi,
                           _s())
    else:
        r = lib.hi_gemv(_p(x), x.stride(0), _p(normw), eps, _p(W), _p(out), out.stride(0), M, N, K, epi, _s())
    _ok(r, "gemv")
    return out


def gemv_qkv_rope(x, W, normw, Hq, Hkv, cs, pos, kc, vc, out, bias=None, eps=1e-5, scales=None):
    """Fused RMSNorm + QKV GEMV (+ bias) + RoPE + KV-cache write. Row m -> cache slot m at pos[m]."""
    D = kc.shape[-1]
    _dev(x, W, cs, pos, kc, vc, out, bias, normw, scales)
    if _w8(W, scales):
        r = lib.hi_gemv_qkv_rope_w8(_p(x), x.stride(0), _p(normw), eps, _p(W), _p(scales), _p(bias), _p(out),
                                    out.stride(0), x.shape[0], x.shape[1], Hq, Hkv, D, _p(cs), _p(pos), _p(kc), _p(vc),
                                    kc.shape[2], _s())
    else:
        r = lib.hi_gemv_qkv_rope(_p(x), x.stride(0), _p(normw), eps, _p(W), _p(bias), _p(out), out.stride(0),
                                 x.shape[0], x.shape[1], Hq, Hkv, D, _p(cs), _p(pos), _p(kc), _p(vc), kc.shape[2], _s())
    _ok(r, "gemv_qkv_rope")
    return out


def gemm(A, W, out=None, epi=0, bias=None, scales=None):
    """C (epi) A[M, K] @ W[N, K]^T on the MFMA GEMM (+ bias for epi 0)."""
    M, K = A.shape
    N = W.shape[0]
    if out is None:
        out = torch.empty(M, N // 2 if epi == 2 else N, dtype=A.dtype, device=A.device)
    _dev(A, W, out, bias, scales)
    if _w8(W, scales):
        r = lib.hi_gemm_w8(_p(A), A.stride(0), _p(W), _p(scales), _p(bias), _p(out), out.stride(0), M, N, K, epi, _s())
    else:
        r = lib.hi_gemm(_p(A), A.stride(0), _p(W), _p(bias), _p(out), out.stride(0), M, N, K, epi, _s())
    _ok(r, "gemm")
    return out


def moe_router(xn, Wr, k, flags):
    """Top-k experts of each normalised row xn [M, H] under router Wr [E, H]: (idx [M, k] int32,
    weights [M, k] fp32), descending."""
    M, H = xn.shape
    _dev(xn, Wr)
    idx = torch.empty(M, k, dtype=torch.int32, device=xn.device)
    w = torch.empty(M, k, dtype=torch.float32, device=xn.device)
    _ok(lib.hi_moe_router(_p(xn), xn.stride(0), _p(Wr), M, Wr.shape[0], H, k, flags, _p(idx), _p(w), _s()), "moe_router")
    return idx, w


def moe_experts(xn, wgu, wdown, idx, w, x, flags, scale=1.0, path=0):
    """x += MoE(xn) in place, given the routing: wgu [E, 2I, H] (gate/up interleaved per expert),
    wdown [E, H, I]. path 0 auto, 1 GEMV, 2 grouped GEMM."""
    M, H = xn.shape
    E, I, k = wgu.shape[0], wdown.shape[2], idx.shape[1]
    _dev(xn, wgu, wdown, idx, w, x)
    work = torch.empty(lib.hi_moe_work_bytes(M, k, E, H, I), dtype=torch.uint8, device=xn.device)
    _ok(lib.hi_moe_experts(_p(xn), xn.stride(0), _p(wgu), _p(wdown), _p(idx), _p(w), M, E, k, H, I, flags, scale, _p(x),
                           x.stride(0), path, _p(work), _s()), "moe_experts")
    return x


def moe_route_experts(xn, Wr, wgu, wdown, k, x, flags, scale=1.0):
    """Router and experts in one call: x += MoE(xn) in place with the routing computed on the way;
    returns (idx [M, k] int32, weights [M, k] fp32) as moe_router would. The same bits as moe_router
    then moe_experts(path=0); up to HIPINFER_GEMV_MAX rows the router runs inside the gate/up launch."""
    M, H = xn.shape
    E, I = wgu.shape[0], wdown.shape[2]
    _dev(xn, Wr, wgu, wdown, x)
    idx = torch.empty(M, k, dtype=torch.int32, device=xn.device)
    w = torch.empty(M, k, dtype=torch.float32, device=xn.device)
    work = torch.empty(lib.hi_moe_work_bytes(M, k, E, H, I), dtype=torch.uint8, device=xn.device)
    _ok(lib.hi_moe_route_experts(_p(xn), xn.stride(0), _p(Wr), _p(wgu), _p(wdown), M, E, k, H, I, flags, scale, _p(x),
                                 x.stride(0), _p(idx), _p(w), _p(work), _s()), "moe_route_experts")
    return idx, w


# ------------------------------------------------------------------ int8 weight format (GPU)
def decode_attn(q, kc, vc, pos, Hq, Hkv, out=None, work=None):
    """Decode attention (reference scripts/hipinfer.py:180-190): q [B, ldq]; kc/vc [B, Hkv, max_seq, D]
    fp16; pos [B] int32 (query b attends to keys 0..pos[b] of cache slot b). work: zeroed once,
    hi_decode_work_bytes(B, Hq, Hkv, D) bytes (the kernel leaves its counters zeroed)."""
    B = q.shape[0]
    D = kc.shape[-1]
    if out is None:
        out = torch.empty(B, Hq * D, dtype=torch.float16, device=q.device)
    if work is None:
        work = torch.zeros(lib.hi_decode_work_bytes(B, Hq, Hkv, D), dtype=torch.uint8, device=q.device)
    _dev(q, kc, vc, pos, out, work)
    _ok(lib.hi_decode_attn(_p(q), q.stride(0), _p(kc), _p(vc), kc.shape[2], _p(pos), _p(out), out.stride(0), B, Hq, Hkv, D,
                           _p(work), _s()), "decode_attn")
    return out


def rope_cache(qkv, Hq, Hkv, cs, kc, vc, pos=None, pos_base=0, slot_base=0):
    """RoPE + KV-cache write after a QKV GEMM (reference scripts/hipinfer.py:164-168): qkv [M,
    (Hq+2Hkv)*D] gets its q heads rotated in place; the rotated k and raw v rows go to kc/vc
    [slots, Hkv, max_seq, D]; cs [max_seq, D/2, 2] fp16. Row m sits at pos[m] in slot
    slot_base + m (decode), or at pos_base + m in slot slot_base (prefill)."""
    D = kc.shape[-1]
    _dev(qkv, cs, kc, vc, pos)
    _ok(lib.hi_rope_cache(_p(qkv), qkv.stride(0), qkv.shape[0], Hq, Hkv, D, _p(cs), _p(pos), pos_base, slot_base,
                          _p(kc), _p(vc), kc.shape[2], _s()), "rope_cache")


def flash_prefill(q, kc, vc, T, p0, Hq, Hkv, out=None):
    """Causal prefill attention (reference scripts/hipinfer.py:171-177): q [T, ldq] with head h at
    columns h*D, row t at position p0 + t; kc/vc [Hkv, max_seq, D] of one cache slot. Returns out
    [T, Hq*D] fp16."""
    D = kc.shape[-1]
    if out is None:
        out = torch.empty(T, Hq * D, dtype=torch.float16, device=q.device)
    _dev(q, kc, vc, out)
    _ok(lib.hi_flash_prefill(_p(q), q.stride(0), _p(kc), _p(vc), kc.shape[1], _p(out), out.stride(0), T, p0, Hq, Hkv,
                             D, _s()), "flash_prefill")
    return out


def flash_prefill_lse(q, kc, vc, T, p0, Hq, Hkv, out=None, lse=None):
    """flash_prefill that also returns each row's log2-domain log-sum-exp, lse [Hq, T] fp32
    (reference scripts/hipinfer.py:193-202)."""
    D = kc.shape[-1]
    if out is None:
        out = torch.empty(T, Hq * D, dtype=torch.float16, device=q.device)
    if lse is None:
        lse = torch.empty(Hq, T, dtype=torch.float32, device=q.device)
    _dev(q, kc, vc, out, lse)
    _ok(lib.hi_flash_prefill_lse(_p(q), q.stride(0), _p(kc), _p(vc), kc.shape[1], _p(out), out.stride(0), T, p0, Hq,
                                 Hkv, D, _p(lse), _s()), "flash_prefill_lse")
    return out, lse


def argmax(logits, out=None):
    """Greedy token per row of logits [B, V] fp16 (reference hi_argmax, api.cu:838): NaN ranks
    highest, ties go to the lowest index, an all -inf row gives 0."""
    B, V = logits.shape
    logits = logits.contiguous()
    if out is None:
        out = torch.empty(B, dtype=torch.int32, device=logits.device)
    _dev(logits, out)
    _ok(lib.hi_argmax(_p(logits), B, V, _p(out), _s()), "argmax")
    return out


def embed(tok, table, out=None):
    """Embedding rows out[b] = table[tok[b]] (the reference engine's embed_kernel)."""
    B = tok.shape[0]
    V, H = table.shape
    if out is None:
        out = torch.empty(B, H, dtype=table.dtype, device=table.device)
    _dev(tok, table, out)
    _ok(lib.hi_embed(_p(tok), _p(table), V, H, _p(out), out.stride(0), B, _s()), "embed")
    return out


def quantize_rows(w):
    """scripts/export.py:54-68 on the GPU, bit-exact: s[n] = fp16(max_k |w[n, k]| / 127),
    q = clamp(round(w / s), -127, 127), q = 0 for an all-zero row. Returns (q int8, s fp16)."""
    assert w.dtype == torch.float16 and w.dim() == 2
    w = w.contiguous()
    _dev(w)
    q = torch.empty(w.shape, dtype=torch.int8, device=w.device)
    s = torch.empty(w.shape[0], dtype=torch.float16, device=w.device)
    _ok(lib.hi_quantize_rows(_p(w), w.shape[0], w.shape[1], _p(q), _p(s), _s()), "quantize_rows")
    return q, s


def dequantize_rows(q, s):
    """scripts/export.py:71-73: fp16(q * s), the weights the int8 GEMM computes with."""
    q = q.contiguous()
    _dev(q, s)
    out = torch.empty(q.shape, dtype=torch.float16, device=q.device)
    _ok(lib.hi_dequantize_rows(_p(q), _p(s), q.shape[0], q.shape[1], _p(out), _s()), "dequantize_rows")
    return out


def interleave_gate_up(gate, up, group=16):
    """scripts/export.py:97-101: [2I, H] with 16 gate rows, then the same 16 up rows, per group."""
    inter, hidden = gate.shape
    g = gate.reshape(inter // group, group, hidden)
    u = up.reshape(inter // group, group, hidden)
    return torch.stack([g, u], dim=1).reshape(2 * inter, hidden)


class Engine:
    """The reference's Engine (scripts/hipinfer.py:334-500) over this library's engine entry
    points, one GPU: a weight file in the export format (versions 2, 3, 4) loaded for max_batch
    slots of max_seq positions, greedy prefill / decode, per-slot token history. tp must be 1.
    Bad arguments raise ValueError (the reason is printed on stderr)."""

    def __init__(self, path, max_batch=8, max_seq=2048, max_prefill=1024, tp=1, devices=None):
        if tp != 1:
            raise ValueError("hipinfer_amd.Engine: one GPU per engine (tp=1)")
        dev = torch.cuda.current_device() if devices is None else list(devices)[0]
        self.tp = 1
        self.device = torch.device("cuda", dev)
        self.h = lib.hi_load_tp(os.fsencode(path), max_batch, max_seq, max_prefill, 1, (C.c_int * 1)(dev))
        if not self.h:
            raise RuntimeError("hi_load failed")
        cfg = (C.c_int * 11)()
        lib.hi_config(self.h, cfg)
        (self.vocab, self.hidden, self.inter, self.layers, self.heads, self.kv_heads, self.head_dim, self.max_pos,
         tied, qkv_bias, self.window) = list(cfg)
        self.tied, self.qkv_bias = bool(tied), bool(qkv_bias)
        moe = (C.c_int * 3)()
        lib.hi_moe_config(self.h, moe)
        self.n_experts, self.top_k, self.moe_flags = list(moe)
        self.quant = lib.hi_weight_quant(self.h)
        self.max_seq, self.max_batch, self.max_prefill = max_seq, max_batch, max_prefill
        self.weight_bytes = lib.hi_weight_bytes(self.h)
        self.kv_bytes_per_token = 2 * self.layers * self.kv_heads * self.head_dim * 2

    @staticmethod
    def _ok(r, what):
        if r < 0:
            raise ValueError(f"hipinfer_amd {what}: bad arguments (see stderr)")
        return r

    def prefill(self, slot, tokens, p0=0):
        arr = (C.c_int * len(tokens))(*tokens)
        return self._ok(lib.hi_prefill(self.h, slot, arr, len(tokens), p0), "prefill")

    def prefill_logits(self, slot, tokens, p0=0):
        """Prefill and return the fp16 logits of every position, [T, vocab] on the GPU."""
        arr = (C.c_int * len(tokens))(*tokens)
        out = torch.empty(len(tokens), self.vocab, dtype=torch.float16, device=self.device)
        self._ok(lib.hi_prefill_logits(self.h, slot, arr, len(tokens), p0, C.c_void_p(out.data_ptr())),
                 "prefill_logits")
        return out

    def decode(self, B, steps, graph=True):
        return self._ok(lib.hi_decode(self.h, B, steps, int(graph)), "decode")

    def history(self, slot, start, n):
        arr = (C.c_int * n)()
        self._ok(lib.hi_history(self.h, slot, start, n, arr), "history")
        return list(arr)

    def logits(self, B):
        out = torch.empty(B, self.vocab, dtype=torch.float16, device=self.device)
        self._ok(lib.hi_logits(self.h, B, C.c_void_p(out.data_ptr())), "logits")
        return out

    def set_state(self, tokens, positions):
        """Next input token and its position for slots [0, len(tokens))."""
        B = len(tokens)
        assert len(positions) == B
        self._ok(lib.hi_set_state(self.h, B, (C.c_int * B)(*tokens), (C.c_int * B)(*positions)), "set_state")

    def rewind(self, slot, length, next_token):
        """Cut slot's cache to `length` positions; the next decode step feeds next_token there."""
        self._ok(lib.hi_rewind(self.h, slot, length, next_token), "rewind")

    MAX_VERIFY = lib.hi_verify_max_rows() if hasattr(lib, "hi_verify_max_rows") else 0

    def verify(self, slot, tokens, p0, graph=True, logits=False):
        """Greedy next token after each of `tokens`, fed at positions p0.. of `slot` (whose cache
        must hold positions < p0), computed by the batch-of-one decode kernels, so entry i is
        exactly the token plain greedy decoding produces at p0 + i given the same prefix. Writes
        the rows' k/v; leaves the slot's next token and position alone (see rewind). With
        logits=True also returns the [len(tokens), vocab] fp16 logits. Dense models."""
        R = len(tokens)
        out = (C.c_int * R)()
        lg = torch.empty(R, self.vocab, dtype=torch.float16, device=self.device) if logits else None
        self._ok(lib.hi_verify(self.h, slot, (C.c_int * R)(*tokens), R, p0, out,
                               None if lg is None else C.c_void_p(lg.data_ptr()), int(graph)), "verify")
        return (list(out), lg) if logits else list(out)

    def generate(self, prompt, n_new, graph=True):
        """Greedy: returns n_new tokens (the first comes from prefill)."""
        first = self.prefill(0, prompt)
        if n_new > 1:
            self.decode(1, n_new - 1, graph)
        return [first] + self.history(0, len(prompt) + 1, n_new - 1)

    def close(self):
        if self.h:
            lib.hi_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
