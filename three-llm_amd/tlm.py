"""ctypes binding of libtlm.so (include/tlm.h).

The library is the only compute path: if it is missing or the device is not
an MI355X (gfx950), every entry point raises.  There is no CPU fallback.
"""
from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Optional

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libtlm.so"

FMT_F16, FMT_Q4, FMT_F32 = 1, 2, 3
(T_EMBED, T_LM_HEAD, T_LM_HEAD_SCALES, T_FINAL_NORM, T_ATTN_NORM, T_FFN_NORM, T_WQKV, T_WQKV_SCALES, T_BQKV, T_WO,
 T_WO_SCALES, T_WGATE, T_WGATE_SCALES, T_WUP, T_WUP_SCALES, T_WDOWN, T_WDOWN_SCALES) = range(17)
LOGITS = 1
# error codes of include/tlm.h
TLM_ERR_INVALID, TLM_ERR_HIP, TLM_ERR_OOM, TLM_ERR_STATE, TLM_ERR_RANGE = -1, -2, -3, -4, -5

# exported symbols (checked by the CPU test suite against include/tlm.h)
EXPORTS = [
    "tlm_abi_version", "tlm_last_error", "tlm_open", "tlm_close", "tlm_sync", "tlm_device_info", "tlm_device_memory",
    "tlm_alloc",
    "tlm_free", "tlm_upload", "tlm_download", "tlm_copy", "tlm_linear_create", "tlm_linear_destroy", "tlm_linear_dequant",
    "tlm_op_linear", "tlm_op_linear_rows", "tlm_op_rmsnorm", "tlm_op_silu_mul", "tlm_op_gated_mlp", "tlm_attn_create", "tlm_attn_destroy",
    "tlm_op_attention", "tlm_op_attention_rows", "tlm_op_attention_rows_noalloc", "tlm_attn_reset", "tlm_attn_read_cache", "tlm_op_logits", "tlm_op_argmax",
    "tlm_op_topk", "tlm_read_candidates",
    "tlm_model_create", "tlm_model_destroy", "tlm_model_upload", "tlm_model_finalize", "tlm_model_set_prefill",
    "tlm_compute_token",
    "tlm_prefill", "tlm_read_logits", "tlm_read_token", "tlm_decode_greedy", "tlm_reset_cache", "tlm_kv_write",
    "tlm_kv_read", "tlm_kv_fill_normal", "tlm_read_hidden", "tlm_time_decode", "tlm_time_kernel", "tlm_time_head",
    "tlm_time_layers", "tlm_trace_decode",
    "tlm_model_describe", "tlm_model_counts_read", "tlm_synth_normal", "tlm_synth_tokens", "tlm_quantize_q4", "tlm_f32_to_f16",
]


class TlmError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(message or f"libtlm error {code}")
        self.code = code


class AttnDesc(ctypes.Structure):
    _fields_ = [("heads", ctypes.c_int32), ("kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("max_tokens", ctypes.c_int32), ("rotary_dim", ctypes.c_int32), ("sliding_window", ctypes.c_int32),
                ("kv_fmt", ctypes.c_int32), ("reserved", ctypes.c_int32), ("inv_freq", ctypes.POINTER(ctypes.c_float)),
                ("attention_factor", ctypes.c_double), ("attn_scale", ctypes.c_double)]


class ModelDesc(ctypes.Structure):
    _fields_ = [("hidden_size", ctypes.c_int32), ("intermediate_size", ctypes.c_int32),
                ("num_layers", ctypes.c_int32), ("num_heads", ctypes.c_int32), ("num_kv_heads", ctypes.c_int32),
                ("head_dim", ctypes.c_int32), ("vocab_size", ctypes.c_int32), ("max_tokens", ctypes.c_int32),
                ("rotary_dim", ctypes.c_int32), ("sliding_window", ctypes.c_int32), ("linear_fmt", ctypes.c_int32),
                ("head_fmt", ctypes.c_int32), ("embed_fmt", ctypes.c_int32), ("kv_fmt", ctypes.c_int32),
                ("qkv_bias", ctypes.c_int32), ("tied", ctypes.c_int32), ("rms_eps", ctypes.c_double),
                ("attention_factor", ctypes.c_double), ("inv_freq", ctypes.POINTER(ctypes.c_float)),
                ("attn_scale", ctypes.c_double), ("layer_windows", ctypes.POINTER(ctypes.c_int32))]


class ModelCounts(ctypes.Structure):
    _fields_ = [("graph_launches", ctypes.c_uint64), ("kernel_launches", ctypes.c_uint64),
                ("prefill_chunks", ctypes.c_uint64), ("replayed_positions", ctypes.c_uint64),
                ("recomputed_positions", ctypes.c_uint64), ("persistent_tokens", ctypes.c_uint64)]


_lib = None
VP = ctypes.c_void_p


def lib():
    """Loads libtlm.so once; raises if it was not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise TlmError(-4, f"three-llm_amd: {LIB_PATH} is missing; build it with "
                               "`python three-llm_amd/build.py` (there is no CPU fallback)")
        L = ctypes.CDLL(str(LIB_PATH))
        i32, u64, sz, dbl = ctypes.c_int32, ctypes.c_uint64, ctypes.c_size_t, ctypes.c_double
        sig = {
            "tlm_abi_version": ([], ctypes.c_int),
            "tlm_last_error": ([], ctypes.c_char_p),
            "tlm_open": ([ctypes.c_int, ctypes.POINTER(VP)], ctypes.c_int),
            "tlm_close": ([VP], None),
            "tlm_sync": ([VP], ctypes.c_int),
            "tlm_device_info": ([VP, ctypes.c_char_p, sz, ctypes.POINTER(ctypes.c_int)], ctypes.c_int),
            "tlm_device_memory": ([VP, ctypes.POINTER(sz), ctypes.POINTER(sz)], ctypes.c_int),
            "tlm_alloc": ([VP, sz, ctypes.POINTER(VP)], ctypes.c_int),
            "tlm_free": ([VP, VP], ctypes.c_int),
            "tlm_upload": ([VP, VP, VP, sz], ctypes.c_int),
            "tlm_download": ([VP, VP, VP, sz], ctypes.c_int),
            "tlm_copy": ([VP, VP, VP, sz], ctypes.c_int),
            "tlm_linear_create": ([VP, ctypes.c_int, ctypes.c_int, ctypes.c_int, VP, VP, ctypes.POINTER(VP)],
                                  ctypes.c_int),
            "tlm_linear_destroy": ([VP], None),
            "tlm_linear_dequant": ([VP, VP], ctypes.c_int),
            "tlm_op_linear": ([VP, VP, VP, VP], ctypes.c_int),
            "tlm_op_linear_rows": ([VP, VP, i32, VP, VP], ctypes.c_int),
            "tlm_op_rmsnorm": ([VP, VP, VP, ctypes.c_int, dbl, ctypes.c_int, VP], ctypes.c_int),
            "tlm_op_silu_mul": ([VP, VP, VP, ctypes.c_int, VP], ctypes.c_int),
            "tlm_op_gated_mlp": ([VP, VP, VP, VP], ctypes.c_int),
            "tlm_attn_create": ([VP, ctypes.POINTER(AttnDesc), ctypes.POINTER(VP)], ctypes.c_int),
            "tlm_attn_destroy": ([VP], None),
            "tlm_op_attention": ([VP, VP, ctypes.c_int, VP], ctypes.c_int),
            "tlm_op_attention_rows": ([VP, VP, i32, i32, VP], ctypes.c_int),
            "tlm_op_attention_rows_noalloc": ([VP, VP, i32, i32, VP], ctypes.c_int),
            "tlm_attn_reset": ([VP], ctypes.c_int),
            "tlm_attn_read_cache": ([VP, ctypes.c_int, VP, VP], ctypes.c_int),
            "tlm_op_logits": ([VP, VP, VP, VP], ctypes.c_int),
            "tlm_op_argmax": ([VP, VP, ctypes.c_int, VP], ctypes.c_int),
            "tlm_op_topk": ([VP, VP, ctypes.c_int, ctypes.c_int, dbl, VP, VP], ctypes.c_int),
            "tlm_read_candidates": ([VP, ctypes.c_int, dbl, VP, VP], ctypes.c_int),
            "tlm_model_create": ([VP, ctypes.POINTER(ModelDesc), ctypes.POINTER(VP)], ctypes.c_int),
            "tlm_model_destroy": ([VP], None),
            "tlm_model_upload": ([VP, ctypes.c_int, ctypes.c_int, VP, sz], ctypes.c_int),
            "tlm_model_finalize": ([VP], ctypes.c_int),
            "tlm_model_set_prefill": ([VP, i32, i32], ctypes.c_int),
            "tlm_compute_token": ([VP, i32, i32, ctypes.c_int], ctypes.c_int),
            "tlm_prefill": ([VP, VP, i32, i32], ctypes.c_int),
            "tlm_read_logits": ([VP, VP, sz], ctypes.c_int),
            "tlm_read_token": ([VP, VP], ctypes.c_int),
            "tlm_decode_greedy": ([VP, i32, i32, ctypes.c_int, VP], ctypes.c_int),
            "tlm_reset_cache": ([VP], ctypes.c_int),
            "tlm_kv_write": ([VP, ctypes.c_int, ctypes.c_int, ctypes.c_int, VP, VP], ctypes.c_int),
            "tlm_kv_read": ([VP, ctypes.c_int, ctypes.c_int, ctypes.c_int, VP, VP], ctypes.c_int),
            "tlm_kv_fill_normal": ([VP, u64, ctypes.c_int], ctypes.c_int),
            "tlm_read_hidden": ([VP, VP, sz], ctypes.c_int),
            "tlm_time_decode": ([VP, i32, i32, ctypes.c_int, ctypes.c_int, ctypes.POINTER(dbl)], ctypes.c_int),
            "tlm_time_kernel": ([VP, ctypes.c_int, ctypes.c_int, ctypes.POINTER(dbl)], ctypes.c_int),
            "tlm_time_head": ([VP, i32, i32, ctypes.c_int, ctypes.POINTER(dbl)], ctypes.c_int),
            "tlm_time_layers": ([VP, i32, i32, ctypes.c_int, ctypes.POINTER(dbl)], ctypes.c_int),
            "tlm_model_describe": ([VP, ctypes.c_char_p, sz], ctypes.c_int),
            "tlm_model_counts_read": ([VP, ctypes.POINTER(ModelCounts)], ctypes.c_int),
            "tlm_trace_decode": ([VP, i32, i32, ctypes.c_int, VP, sz], ctypes.c_int),
            "tlm_synth_normal": ([u64, u64, sz, ctypes.c_float, VP], ctypes.c_int),
            "tlm_synth_tokens": ([u64, u64, sz, i32, VP], ctypes.c_int),
            "tlm_quantize_q4": ([VP, ctypes.c_int, ctypes.c_int, VP, VP], ctypes.c_int),
            "tlm_f32_to_f16": ([VP, sz, VP], ctypes.c_int),
        }
        for name, (args, res) in sig.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = res
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        msg = lib().tlm_last_error()
        raise TlmError(rc, msg.decode() if msg else "")


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(VP)


# ------------------------------------------------------------- host helpers --

def synth_normal(seed: int, stream: int, n: int, std: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    check(lib().tlm_synth_normal(seed, stream, n, std, _ptr(out)))
    return out


def synth_tokens(seed: int, stream: int, n: int, vocab: int) -> np.ndarray:
    out = np.empty(n, np.int32)
    check(lib().tlm_synth_tokens(seed, stream, n, vocab, _ptr(out)))
    return out


def quantize_q4(w: np.ndarray):
    w = np.ascontiguousarray(w, np.float32)
    N, K = w.shape
    packed = np.empty((N, K // 2), np.uint8)
    scales = np.empty((N, K // 32), np.uint16)
    check(lib().tlm_quantize_q4(_ptr(w), N, K, _ptr(packed), _ptr(scales)))
    return packed, scales


def f32_to_f16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    out = np.empty(a.shape, np.uint16)
    check(lib().tlm_f32_to_f16(_ptr(a), a.size, _ptr(out)))
    return out


# ------------------------------------------------------------------ context --

class Buffer:
    """A device allocation owned by a Context."""

    def __init__(self, ctx: "Context", nbytes: int):
        self.ctx = ctx
        self.nbytes = nbytes
        p = VP()
        check(lib().tlm_alloc(ctx.ptr, nbytes, ctypes.byref(p)))
        self.ptr = p

    @property
    def addr(self):
        return self.ptr

    def write(self, a: np.ndarray) -> "Buffer":
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise ValueError("Buffer: write larger than the allocation")
        check(lib().tlm_upload(self.ctx.ptr, self.ptr, _ptr(a), a.nbytes))
        return self

    def read(self, dtype=np.float32, count: Optional[int] = None) -> np.ndarray:
        n = self.nbytes // np.dtype(dtype).itemsize if count is None else count
        out = np.empty(n, dtype)
        check(lib().tlm_download(self.ctx.ptr, _ptr(out), self.ptr, out.nbytes))
        return out

    def copy_from(self, src: "Buffer", nbytes: Optional[int] = None) -> "Buffer":
        """Device-to-device copy on the context stream (asynchronous)."""
        n = min(self.nbytes, src.nbytes) if nbytes is None else nbytes
        check(lib().tlm_copy(self.ctx.ptr, self.ptr, src.ptr, n))
        return self

    def free(self):
        if self.ptr:
            check(lib().tlm_free(self.ctx.ptr, self.ptr))
            self.ptr = None


class Context:
    def __init__(self, device: int = 0):
        p = VP()
        check(lib().tlm_open(device, ctypes.byref(p)))
        self.ptr = p

    def info(self):
        name = ctypes.create_string_buffer(256)
        cus = ctypes.c_int()
        check(lib().tlm_device_info(self.ptr, name, 256, ctypes.byref(cus)))
        return name.value.decode(), cus.value

    def memory(self):
        """(free, total) bytes of device memory."""
        free, total = ctypes.c_size_t(), ctypes.c_size_t()
        check(lib().tlm_device_memory(self.ptr, ctypes.byref(free), ctypes.byref(total)))
        return free.value, total.value

    def buffer(self, nbytes: int) -> Buffer:
        return Buffer(self, nbytes)

    def array(self, a: np.ndarray) -> Buffer:
        a = np.ascontiguousarray(a)
        return Buffer(self, a.nbytes).write(a)

    def sync(self):
        check(lib().tlm_sync(self.ptr))

    def close(self):
        if self.ptr:
            lib().tlm_close(self.ptr)
            self.ptr = None


# -------------------------------------------------------------------- ops --

class Linear:
    """Device-resident weight of TSLLinear (fp16 or q4, [out][in])."""

    def __init__(self, ctx: Context, fmt: int, weights: np.ndarray, scales: Optional[np.ndarray] = None,
                 n_out: Optional[int] = None, k_in: Optional[int] = None):
        self.ctx = ctx
        weights = np.ascontiguousarray(weights)
        if fmt == FMT_Q4:
            n_out, half = weights.shape
            k_in = half * 2
            scales = np.ascontiguousarray(scales, np.uint16)
        else:
            n_out, k_in = weights.shape
        self.n_out, self.k_in, self.fmt = n_out, k_in, fmt
        p = VP()
        check(lib().tlm_linear_create(ctx.ptr, fmt, n_out, k_in, _ptr(weights), _ptr(scales), ctypes.byref(p)))
        self.ptr = p

    def dequant(self) -> np.ndarray:
        out = np.empty((self.n_out, self.k_in), np.float32)
        check(lib().tlm_linear_dequant(self.ptr, _ptr(out)))
        return out

    def __call__(self, x: Buffer, y: Buffer, bias: Optional[Buffer] = None) -> Buffer:
        check(lib().tlm_op_linear(self.ptr, x.ptr, bias.ptr if bias else None, y.ptr))
        return y

    def rows(self, x: Buffer, n_rows: int, y: Buffer, bias: Optional[Buffer] = None) -> Buffer:
        """Batched rows: x fp16 bits [n_rows][k_in] -> y fp32 [n_rows][n_out] (MFMA GEMM)."""
        check(lib().tlm_op_linear_rows(self.ptr, x.ptr, int(n_rows), bias.ptr if bias else None, y.ptr))
        return y

    def close(self):
        if self.ptr:
            lib().tlm_linear_destroy(self.ptr)
            self.ptr = None


class Attention:
    def __init__(self, ctx: Context, heads, kv_heads, head_dim, max_tokens, inv_freq=None, rotary_dim=None,
                 attention_factor=1.0, sliding_window=0, kv_fmt=FMT_F16, attn_scale=0.0):
        self.ctx = ctx
        rd = head_dim if rotary_dim is None else rotary_dim
        if inv_freq is None:
            rd = 0
        self._inv = np.ascontiguousarray(inv_freq if inv_freq is not None else np.zeros(1), np.float32)
        d = AttnDesc(heads, kv_heads, head_dim, max_tokens, rd, sliding_window, kv_fmt, 0,
                     self._inv.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), attention_factor, attn_scale)
        p = VP()
        check(lib().tlm_attn_create(ctx.ptr, ctypes.byref(d), ctypes.byref(p)))
        self.ptr = p
        self.heads, self.kv_heads, self.head_dim, self.max_tokens = heads, kv_heads, head_dim, max_tokens

    def __call__(self, qkv: Buffer, position: int, out: Buffer) -> Buffer:
        check(lib().tlm_op_attention(self.ptr, qkv.ptr, position, out.ptr))
        return out

    def rows(self, qkv: Buffer, n_rows: int, position0: int, out: Buffer) -> Buffer:
        """Positions position0.. at once: qkv fp32 [n_rows][(H+2Hkv)D] -> out fp16 bits [n_rows][H D]."""
        check(lib().tlm_op_attention_rows(self.ptr, qkv.ptr, int(n_rows), int(position0), out.ptr))
        return out

    def rows_noalloc(self, qkv: Buffer, n_rows: int, position0: int, out: Buffer) -> Buffer:
        """rows() through the allocation-free entry point (enqueue only; the
        query staging is the library's fixed 4 MiB device array)."""
        check(lib().tlm_op_attention_rows_noalloc(self.ptr, qkv.ptr, int(n_rows), int(position0), out.ptr))
        return out

    def reset(self):
        check(lib().tlm_attn_reset(self.ptr))

    def read_cache(self, count: int):
        kv = self.kv_heads * self.head_dim
        k = np.empty((count, kv), np.float32)
        v = np.empty((count, kv), np.float32)
        check(lib().tlm_attn_read_cache(self.ptr, count, _ptr(k), _ptr(v)))
        return k, v

    def close(self):
        if self.ptr:
            lib().tlm_attn_destroy(self.ptr)
            self.ptr = None


def rmsnorm(ctx: Context, x: Buffer, w: Optional[Buffer], n: int, eps: float, offset: bool, y: Buffer) -> Buffer:
    check(lib().tlm_op_rmsnorm(ctx.ptr, x.ptr, w.ptr if w else None, n, eps, int(offset), y.ptr))
    return y


def silu_mul(ctx: Context, gate: Buffer, up: Buffer, n: int, out: Buffer) -> Buffer:
    check(lib().tlm_op_silu_mul(ctx.ptr, gate.ptr, up.ptr, n, out.ptr))
    return out


def gated_mlp(gate_up: Linear, down: Linear, x: Buffer, y: Buffer) -> Buffer:
    check(lib().tlm_op_gated_mlp(gate_up.ptr, down.ptr, x.ptr, y.ptr))
    return y


def logits(head: Linear, x: Buffer, out: Optional[Buffer], token: Buffer) -> Buffer:
    check(lib().tlm_op_logits(head.ptr, x.ptr, out.ptr if out else None, token.ptr))
    return token


def argmax(ctx: Context, logits_buf: Buffer, n: int, token: Buffer) -> Buffer:
    check(lib().tlm_op_argmax(ctx.ptr, logits_buf.ptr, n, token.ptr))
    return token


def topk(ctx: Context, logits_buf: Buffer, n: int, k: int, softcap: float = 0.0):
    """TSLLogitSampler candidates: [(token, score)] * k, best first (blocks on the read)."""
    tok, sc = ctx.buffer(4 * k), ctx.buffer(4 * k)
    check(lib().tlm_op_topk(ctx.ptr, logits_buf.ptr, n, k, float(softcap), tok.ptr, sc.ptr))
    t, v = tok.read(np.int32), sc.read(np.float32)
    tok.free()
    sc.free()
    return [(int(a), float(b)) for a, b in zip(t, v)]


# ------------------------------------------------------------------ model --

class Model:
    """Device model: weights, KV cache and the captured per-token graphs."""

    def __init__(self, ctx: Context, desc: ModelDesc, inv_freq: np.ndarray, layer_windows=None):
        """layer_windows: per-layer sliding windows (0 = full causal), or None
        for desc.sliding_window in every layer."""
        self.ctx = ctx
        self._inv = np.ascontiguousarray(inv_freq, np.float32)
        desc.inv_freq = self._inv.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
        if layer_windows is not None:
            self._windows = np.ascontiguousarray(layer_windows, np.int32)
            if self._windows.shape != (desc.num_layers,):
                raise ValueError(f"layer_windows needs {desc.num_layers} entries, got {self._windows.shape}")
            desc.layer_windows = self._windows.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
        self.desc = desc
        p = VP()
        check(lib().tlm_model_create(ctx.ptr, ctypes.byref(desc), ctypes.byref(p)))
        self.ptr = p

    def upload(self, tensor: int, layer: int, a: np.ndarray):
        a = np.ascontiguousarray(a)
        check(lib().tlm_model_upload(self.ptr, tensor, layer, _ptr(a), a.nbytes))

    def finalize(self):
        check(lib().tlm_model_finalize(self.ptr))

    def set_prefill(self, min_rows: int, chunk: int = 2048):
        """Batched (MFMA) prefill for chunks of at least min_rows positions; 0 replays the decode graph."""
        check(lib().tlm_model_set_prefill(self.ptr, int(min_rows), int(chunk)))

    def compute_token(self, token: int, position: int, logits: bool = True):
        check(lib().tlm_compute_token(self.ptr, int(token), int(position), LOGITS if logits else 0))

    def prefill(self, tokens, start: int, end: int):
        t = np.ascontiguousarray(tokens, np.int32).reshape(-1)
        # the library reads tokens[start, end): a shorter array would be read past its end
        if not 0 <= int(start) <= int(end) <= t.size:
            raise TlmError(TLM_ERR_RANGE, f"TLMModel: prefill range [{start}, {end}) outside the "
                                          f"{t.size} tokens given")
        check(lib().tlm_prefill(self.ptr, _ptr(t), int(start), int(end)))

    def read_logits(self, n: Optional[int] = None) -> np.ndarray:
        out = np.empty(self.desc.vocab_size if n is None else n, np.float32)
        check(lib().tlm_read_logits(self.ptr, _ptr(out), out.size))
        return out

    def read_candidates(self, k: int, softcap: float = 0.0):
        """readCandidates: the k best (token, score) of the last logits, best first."""
        t = np.zeros(k, np.int32)
        v = np.zeros(k, np.float32)
        check(lib().tlm_read_candidates(self.ptr, int(k), float(softcap), _ptr(t), _ptr(v)))
        return [(int(a), float(b)) for a, b in zip(t, v)]

    def read_hidden(self) -> np.ndarray:
        out = np.empty(self.desc.hidden_size, np.float32)
        check(lib().tlm_read_hidden(self.ptr, _ptr(out), out.size))
        return out

    def read_token(self) -> int:
        t = np.zeros(1, np.int32)
        check(lib().tlm_read_token(self.ptr, _ptr(t)))
        return int(t[0])

    def decode_greedy(self, token: int, position: int, n: int) -> np.ndarray:
        out = np.zeros(max(n, 1), np.int32)
        check(lib().tlm_decode_greedy(self.ptr, int(token), int(position), int(n), _ptr(out)))
        return out[:n]

    def reset_cache(self):
        check(lib().tlm_reset_cache(self.ptr))

    def kv_write(self, layer: int, pos0: int, k: np.ndarray, v: np.ndarray):
        """k, v: (count, kv_heads, head_dim) in the cache's element type (uint16 fp16
        bits, or float32 for an fp32 cache); the library copies count rows of each."""
        dt = np.float32 if self.desc.kv_fmt == FMT_F32 else np.uint16
        k, v = np.asarray(k), np.asarray(v)
        for name, a in (("k", k), ("v", v)):
            if a.ndim != 3 or a.shape[1:] != (self.desc.num_kv_heads, self.desc.head_dim) or a.dtype != dt:
                raise TlmError(TLM_ERR_INVALID, f"TLMModel: kv_write {name} must be (count, "
                                                f"{self.desc.num_kv_heads}, {self.desc.head_dim}) {np.dtype(dt).name}, "
                                                f"got {a.shape} {a.dtype}")
        if k.shape[0] != v.shape[0]:
            raise TlmError(TLM_ERR_INVALID, f"TLMModel: kv_write k has {k.shape[0]} rows, v {v.shape[0]}")
        check(lib().tlm_kv_write(self.ptr, layer, pos0, k.shape[0], _ptr(np.ascontiguousarray(k)),
                                 _ptr(np.ascontiguousarray(v))))

    def kv_read(self, layer: int, pos0: int, count: int):
        dt = np.float32 if self.desc.kv_fmt == FMT_F32 else np.uint16
        shape = (count, self.desc.num_kv_heads, self.desc.head_dim)
        k = np.empty(shape, dt)
        v = np.empty(shape, dt)
        check(lib().tlm_kv_read(self.ptr, layer, pos0, count, _ptr(k), _ptr(v)))
        return k, v

    def kv_fill_normal(self, seed: int, count: int):
        check(lib().tlm_kv_fill_normal(self.ptr, seed, count))

    def time_decode(self, token: int, position: int, warmup: int, n: int) -> float:
        ms = ctypes.c_double()
        check(lib().tlm_time_decode(self.ptr, int(token), int(position), warmup, n, ctypes.byref(ms)))
        return ms.value

    def time_head(self, token: int, position: int, n: int) -> float:
        """Average ms of the LM head kernel inside n real decode steps."""
        ms = ctypes.c_double()
        check(lib().tlm_time_head(self.ptr, int(token), int(position), n, ctypes.byref(ms)))
        return ms.value

    def time_layers(self, token: int, position: int, n: int) -> float:
        """Average ms of the layer part (the persistent kernel, or the layer
        graph) inside n real decode steps."""
        ms = ctypes.c_double()
        check(lib().tlm_time_layers(self.ptr, int(token), int(position), n, ctypes.byref(ms)))
        return ms.value

    def trace_decode(self, token: int, position: int, n: int, blocks: int) -> np.ndarray:
        """Timeline of the last of n persistent-schedule decode steps:
        uint64 [blocks][16 waves][layers + 1][5 stages][4 events] wall-clock
        stamps (100 MHz)."""
        L = self.desc.num_layers
        out = np.zeros((blocks, 16, L + 1, 5, 4), np.uint64)
        check(lib().tlm_trace_decode(self.ptr, int(token), int(position), int(n), _ptr(out), out.size))
        return out

    def time_kernel(self, which: int, iters: int) -> float:
        ms = ctypes.c_double()
        check(lib().tlm_time_kernel(self.ptr, which, iters, ctypes.byref(ms)))
        return ms.value

    def describe(self) -> str:
        buf = ctypes.create_string_buffer(2048)
        check(lib().tlm_model_describe(self.ptr, buf, 2048))
        return buf.value.decode()

    def counts(self) -> dict:
        """Graph launches, direct kernel launches, batched prefill chunks and
        replayed prompt positions handed to the model's stream so far."""
        c = ModelCounts()
        check(lib().tlm_model_counts_read(self.ptr, ctypes.byref(c)))
        return {name: int(getattr(c, name)) for name, _ in ModelCounts._fields_}

    def close(self):
        if self.ptr:
            lib().tlm_model_destroy(self.ptr)
            self.ptr = None
