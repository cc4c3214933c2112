"""rai_amd: MI355X (gfx950) prompt-lookup decoding and W4A8 kernels.

Python mirror of the `rai_infer` library API for this path (RaiModel,
KVCache, LookupDecoder, LookupConfig, find_ngram_draft, w4a8_matvec,
w4a8_matmul), bound over the C ABI in include/rai_hip.h.  All compute runs in
the HIP library (rai_amd/lib/librai_hip.so); there is no CPU fallback: if the
library is missing or no GPU is present, calls raise.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_size_t, c_uint32, c_uint64, c_void_p
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "librai_hip.so")

RAI_OK = 0
_STATUS = {
    -1: "RAI_E_ARG", -2: "RAI_E_SHAPE", -3: "RAI_E_FORMAT", -4: "RAI_E_OOM", -5: "RAI_E_HIP",
    -6: "RAI_E_WATERMARK", -7: "RAI_E_UNSUPPORTED", -8: "RAI_E_IO", -9: "RAI_E_RANGE",
}


class RaiError(RuntimeError):
    """A failed C-ABI call; `.status` holds the rai_status name."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{_STATUS.get(status, status)}: {message}")
        self.status = _STATUS.get(status, str(status))


class SamplerConfig(ctypes.Structure):
    """rai_sampler_config: SamplerConfig (sampler.rs:17-42) and the repetition
    penalty; the defaults are `rai run`'s (run.rs:40-56)."""
    _fields_ = [("temperature", ctypes.c_float), ("top_k", c_size_t), ("top_p", ctypes.c_float),
                ("repetition_penalty", ctypes.c_float)]

    def __init__(self, temperature=0.7, top_k=40, top_p=0.9, repetition_penalty=1.1):
        super().__init__(temperature, top_k, top_p, repetition_penalty)


class QLinear(ctypes.Structure):
    """rai_qlinear: QuantizedLinear (format.rs:361-367) with device pointers."""
    _fields_ = [("nibbles", c_void_p), ("params", c_void_p), ("rows", c_size_t), ("cols", c_size_t),
                ("group_size", c_size_t)]


class ModelConfig(ctypes.Structure):
    _fields_ = [(n, c_uint32) for n in (
        "hidden_size", "num_layers", "num_heads", "num_kv_heads", "head_dim",
        "intermediate_size", "vocab_size", "max_context")] + [
        ("rope_theta", c_float), ("norm_eps", c_float)] + [
        (n, c_uint32) for n in ("group_size", "embed_group_size", "version", "tied",
                                "num_experts", "experts_per_token", "norm_topk_prob")] + [
        ("embed_scale", c_float), ("attn_scale", c_float)]


class _LookupConfig(ctypes.Structure):
    _fields_ = [("max_draft", c_size_t), ("max_ngram", c_size_t), ("min_ngram", c_size_t),
                ("temperature", c_float)]


class _LookupMatch(ctypes.Structure):
    _fields_ = [("ngram", c_size_t), ("start", c_size_t), ("len", c_size_t)]


class _LookupMetrics(ctypes.Structure):
    _fields_ = [("accepted", c_size_t), ("drafted", c_size_t), ("produced", c_size_t),
                ("matched_ngram", c_size_t), ("accept_rate", c_float)]


class _GenerateStats(ctypes.Structure):
    _fields_ = [(n, c_size_t) for n in ("prompt_tokens", "generated", "steps",
                                        "steps_with_draft", "drafted", "accepted")] + [
        ("prefill_seconds", c_double), ("decode_seconds", c_double)]


class SynthConfig(ctypes.Structure):
    _fields_ = [(n, c_uint32) for n in (
        "hidden_size", "num_layers", "num_heads", "num_kv_heads", "head_dim",
        "intermediate_size", "vocab_size", "max_context")] + [
        ("rope_theta", c_float), ("norm_eps", c_float)] + [
        (n, c_uint32) for n in ("group_size", "embed_group_size", "tied", "num_experts",
                                "experts_per_token", "norm_topk_prob")] + [
        ("weight_std", c_float), ("mode", c_uint32)]


_lib = None


def lib():
    """Load the in-tree HIP library (raises if it is not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: run `python -m rai_amd.build` "
                           "(there is no CPU fallback)")
    L = ctypes.CDLL(LIB_PATH)
    P = c_void_p
    S = c_size_t
    sig = {
        "rai_last_error": (c_char_p, []),
        "rai_device_info": (c_int, [c_char_p, S, POINTER(c_int)]),
        "rai_model_open": (c_int, [c_char_p, c_int, POINTER(c_void_p)]),
        "rai_model_from_buffer": (c_int, [P, S, c_int, POINTER(c_void_p)]),
        "rai_model_free": (None, [P]),
        "rai_model_get_config": (c_int, [P, POINTER(ModelConfig)]),
        "rai_model_weight_bytes": (c_int, [P, POINTER(c_uint64)]),
        "rai_kv_create": (c_int, [P, S, POINTER(c_void_p)]),
        "rai_kv_free": (None, [P]),
        "rai_kv_truncate": (c_int, [P, S]),
        "rai_kv_filled": (c_int, [P, S, POINTER(c_size_t)]),
        "rai_kv_clear": (c_int, [P]),
        "rai_kv_read": (c_int, [P, S, S, S, c_int, P]),
        "rai_embed_token": (c_int, [P, S, P]),
        "rai_forward_from_hidden": (c_int, [P, P, P, S, c_int]),
        "rai_forward_batch": (c_int, [P, P, P, P, S]),
        "rai_hidden_to_logits": (c_int, [P, P, P]),
        "rai_hidden_to_logits_batch": (c_int, [P, P, P, S]),
        "rai_w4a8_matmul_dev": (c_int, [P, P, P, P, S, S, S, S, P]),
        "rai_w4a8_fused_qkv_dev": (c_int, [P, P, P, POINTER(QLinear), POINTER(QLinear), POINTER(QLinear), P, P]),
        "rai_w4a8_fused_gate_up_dev": (c_int, [P, P, POINTER(QLinear), POINTER(QLinear), P, P]),
        "rai_w4a8_matmul_noalloc_dev": (c_int, [P, P, P, P, S, S, S, S, P]),
        "rai_w4a8_lane_sums_dev": (c_int, [P, P, P, S, S, S, S, P]),
        "rai_w4a8_matmul": (c_int, [P, P, P, P, S, S, S, S]),
        "rai_w4a8_time_dev": (c_int, [P, P, P, P, S, S, S, S, S, c_int, POINTER(c_float)]),
        "rai_attention_time_dev": (c_int, [P, P, P, S, S, S, S, S, S, S, c_int, POINTER(c_float)]),
        "rai_tied_lm_head_dev": (c_int, [P, P, P, P, S, S, S, P]),
        "rai_embed_lookup_dev": (c_int, [P, S, P, P, S, S, S, P]),
        "rai_argmax_dev": (c_int, [P, S, S, P, P]),
        "rai_rms_norm_dev": (c_int, [P, P, P, S, S, c_float, P]),
        "rai_silu_mul_dev": (c_int, [P, P, S, S, P]),
        "rai_rope_apply_dev": (c_int, [P, S, S, P, P, P]),
        "rai_attention_head_dev": (c_int, [P, P, P, P, S, S, c_float, P]),
        "rai_find_ngram_draft": (c_int, [P, S, S, S, S, POINTER(_LookupMatch), POINTER(c_int)]),
        "rai_lookup_create": (c_int, [P, S, POINTER(c_void_p)]),
        "rai_lookup_free": (None, [P]),
        "rai_lookup_seed": (c_int, [P, ctypes.c_uint64]),
        "rai_spec_create": (c_int, [P, P, S, POINTER(c_void_p)]),
        "rai_spec_free": (None, [P]),
        "rai_spec_kv": (c_int, [P, c_int, POINTER(c_void_p)]),
        "rai_spec_seed": (c_int, [P, ctypes.c_uint64]),
        "rai_spec_prefill": (c_int, [P, P, S, POINTER(c_size_t)]),
        "rai_spec_step": (c_int, [P, S, ctypes.c_uint32, P, P, S, P]),
        "rai_std_rng_draws": (c_int, [ctypes.c_uint64, P, S, P]),
        "rai_lookup_kv": (c_int, [P, POINTER(c_void_p)]),
        "rai_lookup_prefill": (c_int, [P, P, S, POINTER(c_size_t)]),
        "rai_lookup_step": (c_int, [P, S, P, S, POINTER(_LookupConfig), P, S,
                                    POINTER(_LookupMetrics)]),
        "rai_lookup_generate": (c_int, [P, P, S, S, POINTER(_LookupConfig), P, S,
                                        POINTER(c_size_t), POINTER(_GenerateStats)]),
        "rai_lookup_decode": (c_int, [P, P, S, S, S, POINTER(_LookupConfig), P, S,
                                      POINTER(c_size_t), POINTER(_GenerateStats)]),
        "rai_kv_export": (c_int, [P, S, c_int, P, S]),
        "rai_kv_import": (c_int, [P, S, c_int, P, S]),
        "rai_greedy_generate": (c_int, [P, P, S, S, P]),
        "rai_greedy_decode": (c_int, [P, P, S, S, S, P]),
        "rai_sample_decode": (c_int, [P, P, S, S, S, POINTER(SamplerConfig), P]),
        "rai_sample_tokens": (c_int, [P, S, P, S, POINTER(SamplerConfig), ctypes.c_uint64, S, P]),
        "rai_synth_model": (c_int, [POINTER(SynthConfig), c_uint64, c_char_p,
                                    POINTER(c_void_p), POINTER(c_size_t)]),
        "rai_free_image": (None, [P]),
        "rai_debug_set_attention_spin": (c_int, [c_int]),
        "rai_dev_malloc": (c_int, [S, POINTER(c_void_p)]),
        "rai_dev_free": (c_int, [P]),
        "rai_memcpy_h2d": (c_int, [P, P, S]),
        "rai_memcpy_d2h": (c_int, [P, P, S]),
        "rai_device_synchronize": (c_int, []),
        "rai_stream_create": (c_int, [POINTER(c_void_p)]),
        "rai_stream_destroy": (c_int, [P]),
        "rai_event_create": (c_int, [POINTER(c_void_p)]),
        "rai_event_destroy": (c_int, [P]),
        "rai_event_record": (c_int, [P, P]),
        "rai_event_elapsed_ms": (c_int, [P, P, POINTER(c_float)]),
        "rai_stream_synchronize": (c_int, [P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _check(rc: int) -> None:
    if rc != RAI_OK:
        raise RaiError(rc, lib().rai_last_error().decode())


def _ptr(a: np.ndarray) -> int:
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("array must be C-contiguous")
    return a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint32)


def device_info() -> tuple[str, int]:
    buf = ctypes.create_string_buffer(256)
    cus = c_int()
    _check(lib().rai_device_info(buf, 256, ctypes.byref(cus)))
    return buf.value.decode(), cus.value


def set_attention_spin(polls: int) -> None:
    """Test hook: poll limit of the attention tile hand-off waits (0 = default)."""
    _check(lib().rai_debug_set_attention_spin(polls))


# ---------------------------------------------------------------- device mem --

class DeviceArray:
    """A device allocation owned from Python (plumbing for kernel-level calls)."""

    def __init__(self, nbytes: int):
        p = c_void_p()
        _check(lib().rai_dev_malloc(max(1, nbytes), ctypes.byref(p)))
        self.ptr = p.value
        self.nbytes = nbytes

    @classmethod
    def from_host(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.nbytes)
        if a.nbytes:
            _check(lib().rai_memcpy_h2d(d.ptr, _ptr(a), a.nbytes))
        return d

    def to_host(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype)
        if out.nbytes:
            _check(lib().rai_memcpy_d2h(_ptr(out), self.ptr, out.nbytes))
        return out

    def free(self):
        if self.ptr:
            lib().rai_dev_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ---------------------------------------------------------------- kernels --

def w4a8_matmul(nibbles, params, x, rows: int, cols: int, num_tokens: int,
                group_size: int) -> np.ndarray:
    """w4a8_matmul (gemm.rs:1774-1919): returns out[num_tokens][rows]."""
    nib = np.ascontiguousarray(nibbles, np.uint8)
    par = np.ascontiguousarray(params, np.uint8)
    x = _f32(x)
    out = np.zeros(num_tokens * rows, np.float32)
    _check(lib().rai_w4a8_matmul(_ptr(out), _ptr(nib), _ptr(par), _ptr(x), rows, cols,
                                 num_tokens, group_size))
    return out.reshape(num_tokens, rows)


def w4a8_matvec(nibbles, params, x, rows: int, cols: int, group_size: int) -> np.ndarray:
    """w4a8_matvec (gemm.rs:1336-1384)."""
    return w4a8_matmul(nibbles, params, x, rows, cols, 1, group_size)[0]


def _fused(fn: str, projections, x) -> list[np.ndarray]:
    """Upload each projection (nibbles, params, rows, cols, group_size) and
    the input row, run the fused device entry point, return the outputs."""
    keep, lins, outs = [], [], []
    for nib, par, rows, cols, gs in projections:
        dn = DeviceArray.from_host(np.ascontiguousarray(nib, np.uint8))
        dp = DeviceArray.from_host(np.ascontiguousarray(par, np.uint8))
        keep += [dn, dp]
        lins.append(QLinear(dn.ptr, dp.ptr, rows, cols, gs))
        outs.append(DeviceArray(4 * rows))
    dx = DeviceArray.from_host(_f32(x))
    args = [o.ptr for o in outs] + [ctypes.byref(q) for q in lins] + [dx.ptr, None]
    _check(getattr(lib(), fn)(*args))
    return [o.to_host(np.float32, p[2]) for o, p in zip(outs, projections)]


def sample_tokens(logits, recent, config: SamplerConfig, seed: int, draws: int) -> list[int]:
    """The device sampler alone: apply_repetition_penalty over `recent` then
    sample_token (sampler.rs:47-199), `draws` times from
    StdRng::seed_from_u64(seed)."""
    lg = _f32(np.asarray(logits).reshape(-1))
    r = _u32(recent)
    out = np.zeros(max(draws, 1), np.uint32)
    _check(lib().rai_sample_tokens(_ptr(lg), lg.size, _ptr(r) if r.size else None, r.size, ctypes.byref(config),
                                   seed, draws, _ptr(out)))
    return out[:draws].tolist()


def w4a8_fused_qkv(q, k, v, x) -> list[np.ndarray]:
    """w4a8_fused_qkv (gemm.rs:1386-1557): q, k, v = (nibbles, params, rows,
    cols, group_size) each; returns [q_out, k_out, v_out]."""
    return _fused("rai_w4a8_fused_qkv_dev", [q, k, v], x)


def w4a8_fused_gate_up(gate, up, x) -> list[np.ndarray]:
    """w4a8_fused_gate_up (gemm.rs:1559-1703); returns [gate_out, up_out]."""
    return _fused("rai_w4a8_fused_gate_up_dev", [gate, up], x)


def attention_time(nh: int, nkv: int, hd: int, cap: int, pos: int, m: int, copies: int = 1,
                   iters: int = 20, seed: int = 0) -> tuple[float, float, float]:
    """Average device time (ms) of the attention's score, softmax and PV
    launches for m tokens at positions pos.. over random N(0, 1) K and V
    caches of `cap` positions (HIP events between the launches).  With
    copies > 1 the iterations rotate over that many caches, so that every
    launch streams K and V from HBM."""
    rng = np.random.default_rng(seed)
    vstride = (cap + 63) // 64 * 64
    kn, vn = nkv * cap * hd, nkv * hd * vstride
    q = rng.standard_normal((m, nh * hd), dtype=np.float32)
    kv = rng.standard_normal(max(kn, vn), dtype=np.float32)
    dq, dk, dv = DeviceArray(q.nbytes), DeviceArray(kn * 4 * copies), DeviceArray(vn * 4 * copies)
    _check(lib().rai_memcpy_h2d(c_void_p(dq.ptr), _ptr(q), q.nbytes))
    for c in range(copies):
        _check(lib().rai_memcpy_h2d(c_void_p(dk.ptr + c * kn * 4), _ptr(kv), kn * 4))
        _check(lib().rai_memcpy_h2d(c_void_p(dv.ptr + c * vn * 4), _ptr(kv), vn * 4))
    ms = (c_float * 3)()
    _check(lib().rai_attention_time_dev(dq.ptr, dk.ptr, dv.ptr, cap, pos, m, nh, nkv, hd, copies, iters, ms))
    return ms[0], ms[1], ms[2]


def w4a8_time(nibbles, params, x, rows: int, cols: int, num_tokens: int, group_size: int,
              iters: int = 50, copies: int = 1) -> float:
    """Average device time (ms) of one W4A8 kernel launch (HIP events).
    With copies > 1 the launches rotate over that many device copies of the
    weights (so that, together larger than the last-level cache, every
    launch reads its weights from HBM)."""
    nib = np.ascontiguousarray(nibbles, np.uint8)
    par = np.ascontiguousarray(params, np.uint8)
    dn = DeviceArray(nib.nbytes * copies)
    dp = DeviceArray(par.nbytes * copies)
    for c in range(copies):
        _check(lib().rai_memcpy_h2d(c_void_p(dn.ptr + c * nib.nbytes), _ptr(nib), nib.nbytes))
        _check(lib().rai_memcpy_h2d(c_void_p(dp.ptr + c * par.nbytes), _ptr(par), par.nbytes))
    dx = DeviceArray.from_host(_f32(x))
    do = DeviceArray(num_tokens * rows * 4)
    ms = c_float()
    _check(lib().rai_w4a8_time_dev(do.ptr, dn.ptr, dp.ptr, dx.ptr, rows, cols, num_tokens,
                                   group_size, copies, iters, ctypes.byref(ms)))
    return ms.value


class GemvTimer:
    """rai_w4a8_time_dev over weights uploaded once: `copies` device copies
    of one W4A8 matrix, timed at any number of tokens."""

    def __init__(self, nibbles, params, rows: int, cols: int, group_size: int, copies: int = 1):
        nib = np.ascontiguousarray(nibbles, np.uint8)
        par = np.ascontiguousarray(params, np.uint8)
        self.dn = DeviceArray(nib.nbytes * copies)
        self.dp = DeviceArray(par.nbytes * copies)
        for c in range(copies):
            _check(lib().rai_memcpy_h2d(c_void_p(self.dn.ptr + c * nib.nbytes), _ptr(nib), nib.nbytes))
            _check(lib().rai_memcpy_h2d(c_void_p(self.dp.ptr + c * par.nbytes), _ptr(par), par.nbytes))
        self.rows, self.cols, self.gs, self.copies = rows, cols, group_size, copies

    def time(self, x, num_tokens: int, iters: int = 50) -> float:
        """Average device time (ms) of one launch at num_tokens rows of x."""
        return self.run(x, num_tokens, iters)[0]

    def run(self, x, num_tokens: int, iters: int = 1):
        """(average ms, outputs [num_tokens][rows] of the last launch): the
        launches read the parameters' 16-row tile copy where it applies, as a
        loaded model's batched forward does."""
        dx = DeviceArray.from_host(_f32(x))
        do = DeviceArray(num_tokens * self.rows * 4)
        ms = c_float()
        _check(lib().rai_w4a8_time_dev(do.ptr, self.dn.ptr, self.dp.ptr, dx.ptr, self.rows, self.cols, num_tokens,
                                       self.gs, self.copies, iters, ctypes.byref(ms)))
        return ms.value, do.to_host(np.float32, num_tokens * self.rows).reshape(num_tokens, self.rows)


def w4a8_lane_sums(nibbles, x, rows: int, cols: int, num_tokens: int,
                   group_size: int) -> np.ndarray:
    """Integer accumulators of the W4A8 kernel: [tokens][rows][groups][12]."""
    groups = -(-cols // group_size)
    dn = DeviceArray.from_host(np.ascontiguousarray(nibbles, np.uint8))
    dx = DeviceArray.from_host(_f32(x))
    do = DeviceArray(num_tokens * rows * groups * 12 * 4)
    _check(lib().rai_w4a8_lane_sums_dev(do.ptr, dn.ptr, dx.ptr, rows, cols, num_tokens,
                                        group_size, None))
    return do.to_host(np.int32, num_tokens * rows * groups * 12).reshape(
        num_tokens, rows, groups, 12)


def tied_lm_head(hidden, codes, params, vocab: int, group_size: int) -> np.ndarray:
    """tied_lm_head (gemm.rs:1981-2076)."""
    h = _f32(hidden)
    dh = DeviceArray.from_host(h)
    dc = DeviceArray.from_host(np.ascontiguousarray(codes, np.uint8))
    dp = DeviceArray.from_host(np.ascontiguousarray(params, np.uint8))
    do = DeviceArray(vocab * 4)
    _check(lib().rai_tied_lm_head_dev(do.ptr, dh.ptr, dc.ptr, dp.ptr, vocab, h.size,
                                      group_size, None))
    return do.to_host(np.float32, vocab)


def embed_lookup(token: int, codes, params, vocab: int, hidden: int, group_size: int):
    """embed_lookup (gemm.rs:1926-1970)."""
    dc = DeviceArray.from_host(np.ascontiguousarray(codes, np.uint8))
    dp = DeviceArray.from_host(np.ascontiguousarray(params, np.uint8))
    do = DeviceArray(hidden * 4)
    _check(lib().rai_embed_lookup_dev(do.ptr, token, dc.ptr, dp.ptr, vocab, hidden,
                                      group_size, None))
    return do.to_host(np.float32, hidden)


def argmax(logits) -> np.ndarray:
    """argmax (sampler.rs:201-208) of each row, on the GPU."""
    x = np.atleast_2d(_f32(logits))
    dx = DeviceArray.from_host(x)
    do = DeviceArray(4 * x.shape[0])
    _check(lib().rai_argmax_dev(dx.ptr, x.shape[0], x.shape[1], do.ptr, None))
    return do.to_host(np.uint32, x.shape[0]).astype(np.int64)


def rms_norm(x, weight, eps: float) -> np.ndarray:
    """rms_norm (layers.rs:154-183) of each row of x."""
    x = np.atleast_2d(_f32(x))
    dx, dw = DeviceArray.from_host(x), DeviceArray.from_host(_f32(weight))
    do = DeviceArray(x.nbytes)
    _check(lib().rai_rms_norm_dev(do.ptr, dx.ptr, dw.ptr, x.shape[0], x.shape[1], eps, None))
    _check(lib().rai_device_synchronize())
    return do.to_host(np.float32, x.size).reshape(x.shape)


def silu_mul(gate, up) -> np.ndarray:
    """silu_mul_inplace (layers.rs:824-883) of each row."""
    g = np.atleast_2d(_f32(gate))
    dg, du = DeviceArray.from_host(g), DeviceArray.from_host(np.atleast_2d(_f32(up)))
    _check(lib().rai_silu_mul_dev(dg.ptr, du.ptr, g.shape[0], g.shape[1], None))
    _check(lib().rai_device_synchronize())
    return dg.to_host(np.float32, g.size).reshape(g.shape)


def rope_apply(heads, num_heads: int, head_dim: int, cos_row, sin_row) -> np.ndarray:
    """RoPETable::apply (layers.rs:643-726) for one position."""
    h = _f32(heads)
    dh = DeviceArray.from_host(h)
    dc, ds = DeviceArray.from_host(_f32(cos_row)), DeviceArray.from_host(_f32(sin_row))
    _check(lib().rai_rope_apply_dev(dh.ptr, num_heads, head_dim, dc.ptr, ds.ptr, None))
    _check(lib().rai_device_synchronize())
    return dh.to_host(np.float32, h.size)


def attention_head(q, k, v, pos: int, head_dim: int, scale: float) -> np.ndarray:
    """attention_head (layers.rs:1266-1452) over rows 0..=pos of k and v."""
    dq = DeviceArray.from_host(_f32(q))
    dk = DeviceArray.from_host(_f32(k))
    dv = DeviceArray.from_host(_f32(v))
    do = DeviceArray(head_dim * 4)
    _check(lib().rai_attention_head_dev(do.ptr, dq.ptr, dk.ptr, dv.ptr, pos, head_dim, scale, None))
    _check(lib().rai_device_synchronize())
    return do.to_host(np.float32, head_dim)


@dataclass
class LookupMatch:
    """LookupMatch (lookup.rs:91-109)."""
    ngram: int
    start: int
    len: int

    def draft(self, tokens):
        return list(tokens[self.start:self.start + self.len])


def std_rng_draws(seed: int, kinds) -> np.ndarray:
    """Draws from the device StdRng::seed_from_u64(seed): kinds 0 u32, 1 u64,
    2 f32, 3 f64; returns the raw bits as uint64."""
    k = np.ascontiguousarray(kinds, np.int32)
    out = np.zeros(max(k.size, 1), np.uint64)
    _check(lib().rai_std_rng_draws(seed, _ptr(k), k.size, _ptr(out)))
    return out[:k.size]


def find_ngram_draft(tokens, min_ngram: int, max_ngram: int, max_draft: int):
    """find_ngram_draft (lookup.rs:131-171), evaluated by the GPU search kernel."""
    t = _u32(tokens)
    m = _LookupMatch()
    found = c_int()
    _check(lib().rai_find_ngram_draft(_ptr(t) if t.size else None, t.size, min_ngram,
                                      max_ngram, max_draft, ctypes.byref(m),
                                      ctypes.byref(found)))
    return LookupMatch(m.ngram, m.start, m.len) if found.value else None


# ------------------------------------------------------------------ model --

def synth_model(hidden_size, num_layers, num_heads, num_kv_heads, head_dim,
                intermediate_size, vocab_size, max_context, *, rope_theta=10000.0,
                norm_eps=1e-5, group_size=32, embed_group_size=64, tied=False,
                num_experts=0, experts_per_token=0, norm_topk_prob=False, weight_std=0.02,
                mode=0, seed=0, path: str | None = None) -> np.ndarray | int:
    """Write a random-init .raimodel (see rai_synth_model in include/rai_hip.h).

    Returns the image as a uint8 array, or the file size when `path` is given."""
    c = SynthConfig(hidden_size, num_layers, num_heads, num_kv_heads, head_dim,
                    intermediate_size, vocab_size, max_context, rope_theta, norm_eps,
                    group_size, embed_group_size, int(tied), num_experts, experts_per_token,
                    int(norm_topk_prob), weight_std, mode)
    img = c_void_p()
    n = c_size_t()
    _check(lib().rai_synth_model(ctypes.byref(c), seed, path.encode() if path else None,
                                 ctypes.byref(img), ctypes.byref(n)))
    if path:
        return n.value
    try:
        # numpy buffer filled with memmove (size_t); ctypes.string_at takes a
        # C int size and cannot return images of 2 GiB or more.
        out = np.empty(n.value, np.uint8)
        ctypes.memmove(out.ctypes.data, img.value, n.value)
        return out
    finally:
        lib().rai_free_image(img)


class RaiModel:
    """RaiModel (model.rs:97-1033) resident in HBM."""

    def __init__(self, handle: int):
        self.h = handle
        cfg = ModelConfig()
        _check(lib().rai_model_get_config(self.h, ctypes.byref(cfg)))
        self.config = cfg

    @classmethod
    def load(cls, path: str, max_groups: int = 0) -> "RaiModel":
        h = c_void_p()
        _check(lib().rai_model_open(path.encode(), max_groups, ctypes.byref(h)))
        return cls(h.value)

    @classmethod
    def from_bytes(cls, data, max_groups: int = 0) -> "RaiModel":
        buf = data if isinstance(data, np.ndarray) else np.frombuffer(data, np.uint8)
        buf = np.ascontiguousarray(buf, np.uint8)
        h = c_void_p()
        _check(lib().rai_model_from_buffer(_ptr(buf), buf.size, max_groups, ctypes.byref(h)))
        return cls(h.value)

    def close(self):
        if self.h:
            lib().rai_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def weight_bytes(self) -> int:
        v = c_uint64()
        _check(lib().rai_model_weight_bytes(self.h, ctypes.byref(v)))
        return v.value

    def create_kv_cache(self, max_ctx: int) -> "KVCache":
        h = c_void_p()
        _check(lib().rai_kv_create(self.h, max_ctx, ctypes.byref(h)))
        return KVCache(h.value, owner=self)

    def embed_token(self, token_id: int) -> np.ndarray:
        out = np.zeros(self.config.hidden_size, np.float32)
        _check(lib().rai_embed_token(self.h, token_id, _ptr(out)))
        return out

    def forward_from_hidden(self, hidden, pos: int, kv: "KVCache", store_kv: bool = True):
        h = _f32(hidden).copy()
        _check(lib().rai_forward_from_hidden(self.h, kv.h, _ptr(h), pos, int(store_kv)))
        return h

    def forward_batch(self, hiddens, positions, kv: "KVCache") -> np.ndarray:
        h = _f32(hiddens).copy()
        p = np.ascontiguousarray(positions, np.uint64)
        _check(lib().rai_forward_batch(self.h, kv.h, _ptr(h), _ptr(p), p.size))
        return h

    def hidden_to_logits(self, hidden) -> np.ndarray:
        out = np.zeros(self.config.vocab_size, np.float32)
        h = _f32(hidden)  # kept alive across the call
        _check(lib().rai_hidden_to_logits(self.h, _ptr(h), _ptr(out)))
        return out

    def hidden_to_logits_batch(self, hiddens, batch: int) -> np.ndarray:
        out = np.zeros(batch * self.config.vocab_size, np.float32)
        h = _f32(hiddens)  # kept alive across the call
        _check(lib().rai_hidden_to_logits_batch(self.h, _ptr(h), _ptr(out), batch))
        return out.reshape(batch, self.config.vocab_size)


class KVCache:
    """KVCache (kv_cache.rs:232-330) in HBM."""

    def __init__(self, handle: int, owner=None, borrowed: bool = False):
        self.h = handle
        self._owner = owner
        self._borrowed = borrowed

    def truncate(self, length: int):
        _check(lib().rai_kv_truncate(self.h, length))

    def filled(self, layer: int = 0) -> int:
        v = c_size_t()
        _check(lib().rai_kv_filled(self.h, layer, ctypes.byref(v)))
        return v.value

    def clear(self):
        _check(lib().rai_kv_clear(self.h))

    def get_k(self, layer: int, head: int, pos: int, head_dim: int) -> np.ndarray:
        out = np.zeros(head_dim, np.float32)
        _check(lib().rai_kv_read(self.h, layer, head, pos, 0, _ptr(out)))
        return out

    def get_v(self, layer: int, head: int, pos: int, head_dim: int) -> np.ndarray:
        out = np.zeros(head_dim, np.float32)
        _check(lib().rai_kv_read(self.h, layer, head, pos, 1, _ptr(out)))
        return out

    def export(self, layer: int, which: int, npos: int, num_kv_heads: int, head_dim: int) -> np.ndarray:
        """K (which = 0) or V (1) rows [kv_head][npos][head_dim] of one layer."""
        out = np.zeros((num_kv_heads, npos, head_dim), np.float32)
        _check(lib().rai_kv_export(self.h, layer, which, _ptr(out), npos))
        return out

    def import_rows(self, layer: int, which: int, rows: np.ndarray) -> None:
        """Set one layer's K (which = 0) or V (1) rows [kv_head][npos][head_dim]
        as positions 0..npos; the layer's watermark becomes npos."""
        r = np.ascontiguousarray(rows, np.float32)
        _check(lib().rai_kv_import(self.h, layer, which, _ptr(r), r.shape[1]))

    def __del__(self):
        try:
            if self.h and not self._borrowed:
                lib().rai_kv_free(self.h)
        except Exception:
            pass


@dataclass
class LookupConfig:
    """LookupConfig (lookup.rs:64-89).  temperature > 1e-6 samples exactly
    (lookup.rs:359-403) from the decoder's StdRng; <= 1e-6 is greedy."""
    max_draft: int = 10
    max_ngram: int = 3
    min_ngram: int = 1
    temperature: float = 0.0

    def _c(self) -> _LookupConfig:
        return _LookupConfig(self.max_draft, self.max_ngram, self.min_ngram, self.temperature)


@dataclass
class LookupMetrics:
    """LookupMetrics (lookup.rs:112-119)."""
    accepted: int
    drafted: int
    produced: int
    accept_rate: float
    matched_ngram: int | None


class LookupDecoder:
    """LookupDecoder (lookup.rs:174-455): drafts by n-gram lookup on the GPU,
    verifies [last, draft...] in one batched forward, accepts greedily or by
    exact sampling from its own StdRng (seed with `seed`)."""

    def __init__(self, model: RaiModel, max_ctx: int):
        h = c_void_p()
        _check(lib().rai_lookup_create(model.h, max_ctx, ctypes.byref(h)))
        self.h = h.value
        self.model = model
        kv = c_void_p()
        _check(lib().rai_lookup_kv(self.h, ctypes.byref(kv)))
        self.kv_cache = KVCache(kv.value, owner=self, borrowed=True)

    def seed(self, seed: int) -> None:
        """StdRng::seed_from_u64(seed) for the sampled steps."""
        _check(lib().rai_lookup_seed(self.h, seed))

    def prefill(self, prompt_tokens) -> int:
        p = _u32(prompt_tokens)
        pos = c_size_t()
        _check(lib().rai_lookup_prefill(self.h, _ptr(p), p.size, ctypes.byref(pos)))
        return pos.value

    def step(self, pos: int, context, config: LookupConfig):
        c = _u32(context)
        out = np.zeros(config.max_draft + 1, np.uint32)
        met = _LookupMetrics()
        cfg = config._c()
        _check(lib().rai_lookup_step(self.h, pos, _ptr(c), c.size, ctypes.byref(cfg), _ptr(out),
                                     out.size, ctypes.byref(met)))
        metrics = LookupMetrics(met.accepted, met.drafted, met.produced, met.accept_rate,
                                met.matched_ngram or None)
        return out[:met.produced].tolist(), metrics

    def generate(self, prompt, max_tokens: int, config: LookupConfig):
        """Prefill + step loop in the library (the `rai run` lookup loop)."""
        p = _u32(prompt)
        out = np.zeros(max_tokens + config.max_draft + 1, np.uint32)
        n = c_size_t()
        st = _GenerateStats()
        cfg = config._c()
        _check(lib().rai_lookup_generate(self.h, _ptr(p), p.size, max_tokens, ctypes.byref(cfg),
                                         _ptr(out), out.size, ctypes.byref(n), ctypes.byref(st)))
        stats = {f: getattr(st, f) for f, _ in _GenerateStats._fields_}
        return out[:n.value].tolist(), stats

    def decode(self, context, pos: int, max_tokens: int, config: LookupConfig):
        """The generate loop from a prefilled state (KV holds context[:-1])."""
        c = _u32(context)
        out = np.zeros(max_tokens + config.max_draft + 1, np.uint32)
        n = c_size_t()
        st = _GenerateStats()
        cfg = config._c()
        _check(lib().rai_lookup_decode(self.h, _ptr(c), c.size, pos, max_tokens, ctypes.byref(cfg),
                                       _ptr(out), out.size, ctypes.byref(n), ctypes.byref(st)))
        stats = {f: getattr(st, f) for f, _ in _GenerateStats._fields_}
        return out[:n.value].tolist(), stats

    def greedy_generate(self, prompt, steps: int):
        p = _u32(prompt)
        out = np.zeros(steps, np.uint32)
        _check(lib().rai_greedy_generate(self.h, _ptr(p), p.size, steps, _ptr(out)))
        return out.tolist()

    def sample_decode(self, context, pos: int, steps: int, config: "SamplerConfig"):
        """The `rai run` decode loop without speculation (run.rs:692-735) from a
        prefilled state: repetition penalty + sample_token per token."""
        c = _u32(context)
        out = np.zeros(steps, np.uint32)
        _check(lib().rai_sample_decode(self.h, _ptr(c), c.size, pos, steps, ctypes.byref(config), _ptr(out)))
        return out.tolist()

    def greedy_decode(self, context, pos: int, steps: int):
        """Plain greedy decoding from a prefilled state (KV holds context[:-1])."""
        c = _u32(context)
        out = np.zeros(steps, np.uint32)
        _check(lib().rai_greedy_decode(self.h, _ptr(c), c.size, pos, steps, _ptr(out)))
        return out.tolist()

    def __del__(self):
        try:
            if self.h:
                lib().rai_lookup_free(self.h)
                self.h = None
        except Exception:
            pass


class _SpecConfig(ctypes.Structure):
    _fields_ = [("draft_k", c_size_t), ("temperature", ctypes.c_float)]


class _SpecMetrics(ctypes.Structure):
    _fields_ = [("accepted", c_size_t), ("drafted", c_size_t), ("produced", c_size_t),
                ("accept_rate", ctypes.c_float)]


class SpeculativeDecoder:
    """SpeculativeDecoder (speculative.rs:61-391): a draft model proposes
    draft_k tokens, the target verifies them in one batched forward; exact
    acceptance at temperature > 1e-6 (the decoder's StdRng), greedy below."""

    def __init__(self, draft: RaiModel, target: RaiModel, max_ctx: int):
        h = c_void_p()
        _check(lib().rai_spec_create(draft.h, target.h, max_ctx, ctypes.byref(h)))
        self.h = h.value
        self.draft, self.target = draft, target
        kv0, kv1 = c_void_p(), c_void_p()
        _check(lib().rai_spec_kv(self.h, 0, ctypes.byref(kv0)))
        _check(lib().rai_spec_kv(self.h, 1, ctypes.byref(kv1)))
        self.draft_kv = KVCache(kv0.value, owner=self, borrowed=True)
        self.target_kv = KVCache(kv1.value, owner=self, borrowed=True)

    def seed(self, seed: int) -> None:
        _check(lib().rai_spec_seed(self.h, seed))

    def prefill(self, prompt_tokens) -> int:
        p = _u32(prompt_tokens)
        pos = c_size_t()
        _check(lib().rai_spec_prefill(self.h, _ptr(p), p.size, ctypes.byref(pos)))
        return pos.value

    def step(self, pos: int, last_token: int, draft_k: int, temperature: float = 0.0):
        out = np.zeros(draft_k + 1, np.uint32)
        cfg = _SpecConfig(draft_k, temperature)
        met = _SpecMetrics()
        _check(lib().rai_spec_step(self.h, pos, last_token, ctypes.byref(cfg), _ptr(out), out.size,
                                   ctypes.byref(met)))
        return out[:met.produced].tolist(), {"accepted": met.accepted, "drafted": met.drafted,
                                            "produced": met.produced, "accept_rate": met.accept_rate}

    def __del__(self):
        try:
            if self.h:
                lib().rai_spec_free(self.h)
                self.h = None
        except Exception:
            pass
