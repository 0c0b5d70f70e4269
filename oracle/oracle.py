"""ctypes view of the CPU oracle (oracle/tlm_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker.  The product never imports it.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

F32P = ctypes.POINTER(ctypes.c_float)
U8P = ctypes.POINTER(ctypes.c_uint8)
U16P = ctypes.POINTER(ctypes.c_uint16)

EMBED, LM_HEAD, FINAL_NORM, ATTN_NORM, FFN_NORM, WQKV, BQKV, WO, WGATE, WUP, WDOWN = range(11)


_lib = None


def lib():
    """Loads liboracle.so; raises if it was not built.  It is built by
    `make -C oracle` (or __graft_entry__.build()) before any GPU work: this
    module starts no process, since the tests and the bench call it after the
    GPU is open."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"oracle: {LIB_PATH} is missing; build it with `make -C oracle` "
                               "before running the tests or the bench")
        L = ctypes.CDLL(str(LIB_PATH))
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_bf16_to_f32.restype = ctypes.c_float
        L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f32_to_f16.argtypes = [ctypes.c_float]
        L.orc_linear.argtypes = [F32P, F32P, F32P, ctypes.c_int, ctypes.c_int, F32P]
        L.orc_linear_t.argtypes = [F32P, F32P, F32P, ctypes.c_int, ctypes.c_int, F32P]
        L.orc_rmsnorm.argtypes = [F32P, F32P, ctypes.c_int, ctypes.c_double, ctypes.c_int, F32P]
        L.orc_softmax.argtypes = [F32P, ctypes.c_int, F32P]
        L.orc_silu.restype = ctypes.c_double
        L.orc_silu.argtypes = [ctypes.c_double]
        L.orc_rope_parameters.restype = ctypes.c_int
        L.orc_rope_parameters.argtypes = [ctypes.c_int, ctypes.c_double, ctypes.c_int] + [ctypes.c_double] * 7 + [
            F32P,
            ctypes.POINTER(ctypes.c_double),
        ]
        L.orc_apply_rope.argtypes = [F32P, ctypes.c_int, ctypes.c_int, ctypes.c_int, F32P, ctypes.c_int, ctypes.c_double]
        L.orc_attention.argtypes = [F32P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, F32P, ctypes.c_int,
                                    ctypes.c_double, ctypes.c_double, ctypes.c_int, ctypes.c_int, ctypes.c_int, F32P,
                                    F32P, F32P]
        L.orc_argmax.restype = ctypes.c_int
        L.orc_argmax.argtypes = [F32P, ctypes.c_int]
        L.orc_topk_candidates.argtypes = [F32P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_double,
                                          ctypes.POINTER(ctypes.c_int), F32P]
        L.orc_q4_quantize.argtypes = [F32P, ctypes.c_int, ctypes.c_int, U8P, U16P]
        L.orc_q4_dequant.argtypes = [U8P, U16P, ctypes.c_int, ctypes.c_int, F32P]
        L.orc_model_new.restype = ctypes.c_void_p
        L.orc_model_new.argtypes = [ctypes.c_int] * 8 + [ctypes.c_double, ctypes.c_int, F32P, ctypes.c_int,
                                                         ctypes.c_double, ctypes.c_int, ctypes.c_int]
        L.orc_model_set.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, F32P]
        L.orc_model_set_attention.argtypes = [ctypes.c_void_p, ctypes.c_double, ctypes.POINTER(ctypes.c_int)]
        L.orc_model_free.argtypes = [ctypes.c_void_p]
        L.orc_model_reset.argtypes = [ctypes.c_void_p]
        L.orc_model_read_cache.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, F32P, F32P]
        L.orc_model_write_cache.restype = ctypes.c_int
        L.orc_model_write_cache.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, F32P, F32P]
        L.orc_forward_token.restype = ctypes.c_int
        L.orc_forward_token.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, F32P, F32P]
        L.orc_set_threads.argtypes = [ctypes.c_int]
        _lib = L
    return _lib


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(F32P)


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def f16_to_f32(bits: int) -> float:
    return lib().orc_f16_to_f32(bits)


def bf16_to_f32(bits: int) -> float:
    return lib().orc_bf16_to_f32(bits)


def f32_to_f16(value: float) -> int:
    return lib().orc_f32_to_f16(value)


def linear(x, w, bias, n_in, n_out):
    """runtime/math.ts:6-25 with W [in][out]."""
    x, xp = _f32(x)
    w, wp = _f32(w)
    b, bp = (None, None) if bias is None else _f32(bias)
    y = np.zeros(n_out, np.float32)
    lib().orc_linear(xp, wp, bp, n_in, n_out, y.ctypes.data_as(F32P))
    return y


def linear_t(x, wt, bias=None):
    """Same reduction with W stored [out][in]."""
    x, xp = _f32(x)
    wt, wp = _f32(wt)
    n_out, n_in = wt.shape
    b, bp = (None, None) if bias is None else _f32(bias)
    y = np.zeros(n_out, np.float32)
    lib().orc_linear_t(xp, wp, bp, n_in, n_out, y.ctypes.data_as(F32P))
    return y


def rmsnorm(x, w, eps=1e-5, offset=False):
    x, xp = _f32(x)
    w, wp = (None, None) if w is None else _f32(w)
    y = np.zeros(len(x), np.float32)
    lib().orc_rmsnorm(xp, wp, len(x), eps, int(offset), y.ctypes.data_as(F32P))
    return y


def softmax(v):
    v, vp = _f32(v)
    y = np.zeros(len(v), np.float32)
    lib().orc_softmax(vp, len(v), y.ctypes.data_as(F32P))
    return y


def silu(x: float) -> float:
    return lib().orc_silu(x)


ROPE_KINDS = {None: 0, "default": 0, "linear": 1, "yarn": 2, "llama3": 3}


def rope_parameters(dim, theta, scaling=None):
    """runtime/rope.ts:4-52.  scaling: dict in the reference's RopeScalingConfig
    shape ({type, factor, originalContextLength, betaFast, betaSlow,
    attentionFactor, lowFreqFactor, highFreqFactor}) or None."""
    s = scaling or {}
    kind = ROPE_KINDS[s.get("type")]
    inv = np.zeros(max(dim // 2, 1), np.float32)
    af = ctypes.c_double(0)
    rc = lib().orc_rope_parameters(
        dim, float(theta), kind, float(s.get("factor", 1.0)), float(s.get("originalContextLength", 0)),
        float(s.get("betaFast", 32)), float(s.get("betaSlow", 1)),
        float(s["attentionFactor"]) if s.get("attentionFactor") is not None else -1.0,
        float(s.get("lowFreqFactor", 0)), float(s.get("highFreqFactor", 0)),
        inv.ctypes.data_as(F32P), ctypes.byref(af))
    if rc != 0:
        raise ValueError("oracle: invalid RoPE parameters")
    return inv[: dim // 2], af.value


def apply_rope(v, rotary_dim, position, inv_freq, attention_factor=1.0, pair_count=None, head_offset=0):
    v = np.array(v, dtype=np.float32, copy=True)
    inv, ip = _f32(inv_freq)
    lib().orc_apply_rope(v.ctypes.data_as(F32P), head_offset, rotary_dim, position, ip,
                         rotary_dim // 2 if pair_count is None else pair_count, attention_factor)
    return v


def attention(qkv, heads, kv_heads, head_dim, position, k_cache, v_cache, inv_freq, rotary_dim=None,
              attention_factor=1.0, sliding_window=0, kv_f16=False, attn_scale=0.0):
    """One causalAttention call (runtime/math.ts:179-276); caches are updated in place."""
    rd = head_dim if rotary_dim is None else rotary_dim
    qkv, qp = _f32(qkv)
    inv, ip = _f32(inv_freq)
    assert k_cache.dtype == np.float32 and k_cache.flags.c_contiguous
    out = np.zeros(heads * head_dim, np.float32)
    lib().orc_attention(qp, heads, kv_heads, head_dim, rd, ip, rd // 2, attention_factor, attn_scale,
                        sliding_window, int(kv_f16), position, k_cache.ctypes.data_as(F32P),
                        v_cache.ctypes.data_as(F32P), out.ctypes.data_as(F32P))
    return out


def argmax(logits) -> int:
    logits, lp = _f32(logits)
    return lib().orc_argmax(lp, len(logits))


def topk_candidates(logits, k, chunk=8192, softcap=0.0):
    """TSLLogitSampler candidates: [(token, score)] * k, best first."""
    lg, lp = _f32(logits)
    t = np.zeros(k, np.int32)
    v = np.zeros(k, np.float32)
    lib().orc_topk_candidates(lp, len(lg), int(chunk), int(k), float(softcap or 0.0),
                              t.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), v.ctypes.data_as(F32P))
    return [(int(a), float(b)) for a, b in zip(t, v)]


def q4_quantize(w):
    w, wp = _f32(w)
    N, K = w.shape
    packed = np.zeros((N, K // 2), np.uint8)
    scales = np.zeros((N, K // 32), np.uint16)
    lib().orc_q4_quantize(wp, N, K, packed.ctypes.data_as(U8P), scales.ctypes.data_as(U16P))
    return packed, scales


def q4_dequant(packed, scales):
    packed = np.ascontiguousarray(packed, np.uint8)
    scales = np.ascontiguousarray(scales, np.uint16)
    N, half = packed.shape
    K = half * 2
    out = np.zeros((N, K), np.float32)
    lib().orc_q4_dequant(packed.ctypes.data_as(U8P), scales.ctypes.data_as(U16P), N, K, out.ctypes.data_as(F32P))
    return out


class Model:
    """CPU decoder (DecoderCPURunner restated).  Weights are fp32 [out][in]
    numpy arrays; the object keeps references so the C side may borrow them."""

    def __init__(self, hidden, inter, layers, heads, kv_heads, head_dim, vocab, max_tokens, eps, inv_freq,
                 attention_factor=1.0, rotary_dim=None, sliding_window=0, kv_f16=False, attn_scale=0.0,
                 layer_windows=None):
        self.dims = dict(hidden=hidden, inter=inter, layers=layers, heads=heads, kv_heads=kv_heads,
                         head_dim=head_dim, vocab=vocab, max_tokens=max_tokens)
        rd = head_dim if rotary_dim is None else rotary_dim
        inv, ip = _f32(inv_freq)
        self._keep = [inv]
        self.ptr = lib().orc_model_new(hidden, inter, layers, heads, kv_heads, head_dim, vocab, max_tokens, eps, rd,
                                       ip, rd // 2, attention_factor, sliding_window, int(kv_f16))
        if attn_scale or layer_windows is not None:
            wins = None
            if layer_windows is not None:
                wins = np.ascontiguousarray(layer_windows, np.int32)
                if wins.shape != (layers,) or (wins < 0).any():
                    raise ValueError("oracle: layer_windows needs one non-negative window per layer")
            lib().orc_model_set_attention(self.ptr, float(attn_scale),
                                          wins.ctypes.data_as(ctypes.POINTER(ctypes.c_int)) if wins is not None
                                          else None)

    def set(self, tensor, layer, data):
        if data is None:
            return
        arr, p = _f32(data)
        self._keep.append(arr)
        lib().orc_model_set(self.ptr, tensor, layer, p)

    def reset(self):
        lib().orc_model_reset(self.ptr)

    def read_cache(self, layer, count):
        kv = self.dims["kv_heads"] * self.dims["head_dim"]
        k = np.zeros((count, kv), np.float32)
        v = np.zeros((count, kv), np.float32)
        lib().orc_model_read_cache(self.ptr, layer, count, k.ctypes.data_as(F32P), v.ctypes.data_as(F32P))
        return k, v

    def write_cache(self, layer, pos0, k, v):
        """Cache rows [pos0, pos0 + count) of one layer, (count, kv_heads, head_dim)
        or (count, kv_heads * head_dim) fp32 (e.g. a device cache widened)."""
        kv = self.dims["kv_heads"] * self.dims["head_dim"]
        k = np.ascontiguousarray(np.asarray(k, np.float32).reshape(-1, kv))
        v = np.ascontiguousarray(np.asarray(v, np.float32).reshape(-1, kv))
        assert k.shape == v.shape
        if lib().orc_model_write_cache(self.ptr, int(layer), int(pos0), k.shape[0], k.ctypes.data_as(F32P),
                                       v.ctypes.data_as(F32P)) != 0:
            raise ValueError("oracle: cache rows out of range")

    def forward(self, token, position, want_hidden=False):
        logits = np.zeros(self.dims["vocab"], np.float32)
        hidden = np.zeros(self.dims["hidden"], np.float32) if want_hidden else None
        rc = lib().orc_forward_token(self.ptr, int(token), int(position), logits.ctypes.data_as(F32P),
                                     hidden.ctypes.data_as(F32P) if want_hidden else None)
        if rc != 0:
            raise ValueError("oracle: token or position out of range")
        return (logits, hidden) if want_hidden else logits

    def prefill(self, token, position):
        """One prompt position without the LM head (prefillTokens computes no
        logits, DecoderTSLRunner.ts:504-530)."""
        if lib().orc_forward_token(self.ptr, int(token), int(position), None, None) != 0:
            raise ValueError("oracle: token or position out of range")

    def close(self):
        if self.ptr:
            lib().orc_model_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
