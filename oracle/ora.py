"""ctypes binding for the CPU oracle (oracle/build/liboracle.so).

TEST INFRASTRUCTURE ONLY: the oracle is a C++ restatement of rai's AVX2 CPU
path used to check the HIP library and to time the CPU baseline.  Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
import this module.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_double, c_float, c_int, c_int64, c_size_t, c_uint32, c_uint64, c_void_p

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "build", "liboracle.so")


class OracleConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "hidden_size", "num_layers", "num_heads", "num_kv_heads", "head_dim",
        "intermediate_size", "vocab_size", "max_context")] + [
        ("rope_theta", c_float), ("norm_eps", c_float)] + [
        (n, ctypes.c_uint32) for n in (
            "group_size", "embed_group_size", "version", "tied", "num_experts",
            "experts_per_token", "norm_topk_prob")] + [
        ("embed_scale", c_float), ("attn_scale", c_float)]


class OracleMetrics(ctypes.Structure):
    _fields_ = [("accepted", ctypes.c_int32), ("drafted", ctypes.c_int32),
                ("produced", ctypes.c_int32), ("matched_ngram", ctypes.c_int32)]


_lib = None


def build() -> None:
    import subprocess
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    L = ctypes.CDLL(LIB_PATH)
    P = c_void_p
    sig = {
        "ora_set_threads": (None, [c_int]),
        "ora_get_threads": (c_int, []),
        "ora_last_error": (ctypes.c_char_p, []),
        "ora_quantize_split": (c_int, [P, c_int, c_int, P, P, P]),
        "ora_input_sums": (c_int, [P, c_int, c_int, P]),
        "ora_w4a8_matvec": (c_int, [P, P, P, P, c_int, c_int, c_int]),
        "ora_w4a8_matmul": (c_int, [P, P, P, P, c_int, c_int, c_int, c_int]),
        "ora_w4a8_lane_sums": (c_int, [P, P, P, c_int, c_int, c_int, c_int]),
        "ora_tied_lm_head": (c_int, [P, P, P, P, c_int, c_int, c_int]),
        "ora_embed_lookup": (c_int, [P, c_int, P, P, c_int, c_int, c_int]),
        "ora_rms_norm": (c_int, [P, P, P, c_int, c_float]),
        "ora_rms_norm_residual": (c_int, [P, P, P, P, c_int, c_float]),
        "ora_silu_mul": (c_int, [P, P, c_int]),
        "ora_rope_tables": (c_int, [P, P, c_int, c_int, c_float]),
        "ora_rope_apply": (c_int, [P, c_int, c_int, P, P]),
        "ora_attention_head": (c_int, [P, P, P, c_int, c_int, c_float, P]),
        "ora_expf": (c_float, [c_float]),
        "ora_schraudolph": (c_float, [c_float]),
        "ora_argmax": (c_int64, [P, c_int64]),
        "ora_find_ngram_draft": (c_int, [P, c_int64, c_int64, c_int64, c_int64, P]),
        "ora_model_open": (c_int, [P, c_size_t, c_int, POINTER(c_void_p)]),
        "ora_model_free": (None, [P]),
        "ora_model_config": (c_int, [P, POINTER(OracleConfig)]),
        "ora_kv_create": (c_int, [P, c_int, POINTER(c_void_p)]),
        "ora_kv_free": (None, [P]),
        "ora_kv_truncate": (c_int, [P, c_int]),
        "ora_kv_filled": (c_int, [P, c_int]),
        "ora_kv_read": (c_int, [P, c_int, c_int, c_int, c_int, P]),
        "ora_kv_import": (c_int, [P, c_int, c_int, P, c_int]),
        "ora_lookup_decode_one": (c_int, [P, c_int, c_int, P]),
        "ora_lookup_decode_sample": (c_int, [P, c_int, c_int, P, c_int, c_float, c_int64, c_float, c_float, P, P]),
        "ora_sample_plain": (c_int, [P, c_int, P, c_int, c_float, c_int64, c_float, c_float, P, POINTER(c_int)]),
        "ora_route_experts": (c_int, [P, P, c_int, c_int, c_int, c_int, P, P]),
        "ora_embed_token": (c_int, [P, c_int, P]),
        "ora_forward_from_hidden": (c_int, [P, P, P, c_int, c_int]),
        "ora_forward_batch": (c_int, [P, P, P, P, c_int]),
        "ora_hidden_to_logits": (c_int, [P, P, P]),
        "ora_hidden_to_logits_batch": (c_int, [P, P, P, c_int]),
        "ora_lookup_create": (c_int, [P, c_int, POINTER(c_void_p)]),
        "ora_lookup_free": (None, [P]),
        "ora_lookup_prefill": (c_int, [P, P, c_int, POINTER(c_int)]),
        "ora_lookup_step_greedy": (c_int, [P, c_int, P, c_int, c_int, c_int, c_int, P,
                                           POINTER(OracleMetrics)]),
        "ora_lookup_kv_filled": (c_int, [P]),
        "ora_lookup_import_kv": (c_int, [P, c_int, c_int, P, c_int]),
        "ora_greedy_generate": (c_int, [P, P, c_int, c_int, c_int, P]),
        "ora_chacha_block": (c_int, [P, c_uint64, c_uint64, c_int, P]),
        "ora_rng_create": (c_int, [c_uint64, c_int, P, POINTER(c_void_p)]),
        "ora_rng_free": (None, [P]),
        "ora_rng_next_u32": (c_uint32, [P]),
        "ora_rng_next_u64": (c_uint64, [P]),
        "ora_rng_gen_f32": (c_float, [P]),
        "ora_rng_gen_f64": (c_double, [P]),
        "ora_standard_f32": (c_float, [ctypes.c_uint32]),
        "ora_standard_f64": (c_double, [ctypes.c_uint64]),
        "ora_rng_key": (None, [P, P]),
        "ora_softmax_probabilities": (c_int, [P, c_int, c_float, P]),
        "ora_sample_token": (c_int, [P, c_int, c_float, P, POINTER(c_int)]),
        "ora_sampled_accept": (c_int, [P, c_int, P, c_int, c_float, P, P, POINTER(c_int), POINTER(c_int)]),
        "ora_spec_accept": (c_int, [P, P, c_int, P, c_int, c_float, P, P, POINTER(c_int), POINTER(c_int)]),
        "ora_spec_create": (c_int, [P, P, c_int, POINTER(c_void_p)]),
        "ora_spec_free": (None, [P]),
        "ora_spec_prefill": (c_int, [P, P, c_int, POINTER(c_int)]),
        "ora_spec_step": (c_int, [P, c_int, c_int, c_int, c_float, P, P, POINTER(OracleMetrics)]),
        "ora_lookup_step_sampled": (c_int, [P, c_int, P, c_int, c_int, c_int, c_int, c_float, P, P,
                                            POINTER(OracleMetrics)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


class OracleError(RuntimeError):
    pass


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _check(rc: int) -> None:
    if rc != 0:
        raise OracleError(lib().ora_last_error().decode())


def set_threads(n: int) -> None:
    lib().ora_set_threads(n)


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def w4a8_matmul(nib, params, x, rows, cols, m, gs) -> np.ndarray:
    nib = np.ascontiguousarray(nib, np.uint8)
    params = np.ascontiguousarray(params, np.uint8)
    x = f32(x)
    out = np.zeros(m * rows, np.float32)
    _check(lib().ora_w4a8_matmul(_ptr(out), _ptr(nib), _ptr(params), _ptr(x), rows, cols, m, gs))
    return out.reshape(m, rows)


def w4a8_matvec(nib, params, x, rows, cols, gs) -> np.ndarray:
    nib = np.ascontiguousarray(nib, np.uint8)
    params = np.ascontiguousarray(params, np.uint8)
    x = f32(x)
    out = np.zeros(rows, np.float32)
    _check(lib().ora_w4a8_matvec(_ptr(out), _ptr(nib), _ptr(params), _ptr(x), rows, cols, gs))
    return out


def lane_sums(nib, x, rows, cols, m, gs) -> np.ndarray:
    nib = np.ascontiguousarray(nib, np.uint8)
    x = f32(x)
    groups = -(-cols // gs)
    out = np.zeros(m * rows * groups * 12, np.int32)
    _check(lib().ora_w4a8_lane_sums(_ptr(out), _ptr(nib), _ptr(x), rows, cols, m, gs))
    return out.reshape(m, rows, groups, 12)


def quantize_split(x, gs):
    x = f32(x)
    cols = x.size
    qe = np.zeros(cols // 2, np.int8)
    qo = np.zeros(cols // 2, np.int8)
    sc = np.zeros(-(-cols // gs), np.float32)
    _check(lib().ora_quantize_split(_ptr(x), cols, gs, _ptr(qe), _ptr(qo), _ptr(sc)))
    return qe, qo, sc


def input_sums(x, gs):
    x = f32(x)
    out = np.zeros(-(-x.size // gs), np.float32)
    _check(lib().ora_input_sums(_ptr(x), x.size, gs, _ptr(out)))
    return out


def tied_lm_head(hidden, codes, params, vocab, gs):
    hidden = f32(hidden)
    codes = np.ascontiguousarray(codes, np.uint8)
    params = np.ascontiguousarray(params, np.uint8)
    out = np.zeros(vocab, np.float32)
    _check(lib().ora_tied_lm_head(_ptr(out), _ptr(hidden), _ptr(codes), _ptr(params), vocab,
                                  hidden.size, gs))
    return out


def embed_lookup(token, codes, params, vocab, hidden, gs):
    codes = np.ascontiguousarray(codes, np.uint8)
    params = np.ascontiguousarray(params, np.uint8)
    out = np.zeros(hidden, np.float32)
    _check(lib().ora_embed_lookup(_ptr(out), token, _ptr(codes), _ptr(params), vocab, hidden, gs))
    return out


def rms_norm(x, w, eps):
    x, w = f32(x), f32(w)
    out = np.zeros_like(x)
    _check(lib().ora_rms_norm(_ptr(out), _ptr(x), _ptr(w), x.size, eps))
    return out


def silu_mul(gate, up):
    g = f32(gate).copy()
    u = f32(up)
    _check(lib().ora_silu_mul(_ptr(g), _ptr(u), g.size))
    return g


def rope_tables(head_dim, max_ctx, theta):
    c = np.zeros(max_ctx * (head_dim // 2), np.float32)
    s = np.zeros_like(c)
    _check(lib().ora_rope_tables(_ptr(c), _ptr(s), head_dim, max_ctx, theta))
    return c.reshape(max_ctx, head_dim // 2), s.reshape(max_ctx, head_dim // 2)


def rope_apply(heads, num_heads, head_dim, cos_row, sin_row):
    h = f32(heads).copy()
    c, s = f32(cos_row), f32(sin_row)  # kept alive across the call
    _check(lib().ora_rope_apply(_ptr(h), num_heads, head_dim, _ptr(c), _ptr(s)))
    return h


def attention_head(q, k, v, pos, head_dim, scale):
    q, k, v = f32(q), f32(k), f32(v)
    out = np.zeros(head_dim, np.float32)
    _check(lib().ora_attention_head(_ptr(q), _ptr(k), _ptr(v), pos, head_dim, scale, _ptr(out)))
    return out


def expf(x: float) -> float:
    return lib().ora_expf(x)


def schraudolph(x: float) -> float:
    return lib().ora_schraudolph(x)


def argmax(v) -> int:
    v = f32(v)
    return int(lib().ora_argmax(_ptr(v), v.size))


def route_experts(router, x, num_experts, topk, norm_topk_prob=False):
    """route_experts (layers.rs:1808-1870): (experts, weights) of one token."""
    router, x = f32(router), f32(x)
    sel = np.zeros(topk, np.int32)
    wts = np.zeros(topk, np.float32)
    _check(lib().ora_route_experts(_ptr(router), _ptr(x), x.size, num_experts, topk,
                                   int(norm_topk_prob), _ptr(sel), _ptr(wts)))
    return sel, wts


def find_ngram_draft(tokens, min_ngram, max_ngram, max_draft):
    t = np.ascontiguousarray(tokens, np.int32)
    res = np.zeros(3, np.int64)
    hit = lib().ora_find_ngram_draft(_ptr(t) if t.size else None, t.size, min_ngram, max_ngram,
                                     max_draft, _ptr(res))
    return (int(res[0]), int(res[1]), int(res[2])) if hit else None


class Model:
    """Oracle counterpart of RaiModel (model.rs) over an in-memory .raimodel."""

    def __init__(self, data: bytes | np.ndarray, max_groups: int = 0):
        buf = data if isinstance(data, np.ndarray) else np.frombuffer(bytes(data), np.uint8)
        buf = np.ascontiguousarray(buf, np.uint8)
        h = c_void_p()
        _check(lib().ora_model_open(_ptr(buf), buf.size, max_groups, ctypes.byref(h)))
        self.h = h
        cfg = OracleConfig()
        _check(lib().ora_model_config(h, ctypes.byref(cfg)))
        self.cfg = cfg

    def close(self):
        if self.h:
            lib().ora_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def create_kv(self, max_ctx: int) -> "KVCache":
        return KVCache(self, max_ctx)

    def embed_token(self, token: int) -> np.ndarray:
        out = np.zeros(self.cfg.hidden_size, np.float32)
        _check(lib().ora_embed_token(self.h, token, _ptr(out)))
        return out

    def forward_from_hidden(self, hidden, pos, kv):
        h = f32(hidden).copy()
        _check(lib().ora_forward_from_hidden(self.h, kv.h, _ptr(h), pos, 1))
        return h

    def forward_batch(self, hiddens, positions, kv):
        h = f32(hiddens).copy()
        p = np.ascontiguousarray(positions, np.int32)
        _check(lib().ora_forward_batch(self.h, kv.h, _ptr(h), _ptr(p), p.size))
        return h

    def hidden_to_logits(self, hidden):
        out = np.zeros(self.cfg.vocab_size, np.float32)
        h = f32(hidden)  # kept alive across the call
        _check(lib().ora_hidden_to_logits(self.h, _ptr(h), _ptr(out)))
        return out

    def hidden_to_logits_batch(self, hiddens, batch):
        out = np.zeros(batch * self.cfg.vocab_size, np.float32)
        h = f32(hiddens)  # kept alive across the call
        _check(lib().ora_hidden_to_logits_batch(self.h, _ptr(h), _ptr(out), batch))
        return out.reshape(batch, self.cfg.vocab_size)

    def greedy_generate(self, prompt, steps, max_ctx):
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.zeros(steps, np.int32)
        _check(lib().ora_greedy_generate(self.h, _ptr(p), p.size, steps, max_ctx, _ptr(out)))
        return out


class KVCache:
    def __init__(self, model: Model, max_ctx: int):
        h = c_void_p()
        _check(lib().ora_kv_create(model.h, max_ctx, ctypes.byref(h)))
        self.h = h

    def truncate(self, n: int):
        _check(lib().ora_kv_truncate(self.h, n))

    def filled(self, layer: int = 0) -> int:
        return lib().ora_kv_filled(self.h, layer)

    def get_k(self, layer: int, head: int, pos: int, head_dim: int) -> np.ndarray:
        out = np.zeros(head_dim, np.float32)
        _check(lib().ora_kv_read(self.h, layer, head, pos, 0, _ptr(out)))
        return out

    def get_v(self, layer: int, head: int, pos: int, head_dim: int) -> np.ndarray:
        out = np.zeros(head_dim, np.float32)
        _check(lib().ora_kv_read(self.h, layer, head, pos, 1, _ptr(out)))
        return out

    def import_rows(self, layer: int, which: int, rows: np.ndarray) -> None:
        """Set one layer's K (0) or V (1) rows [nkv][npos][head_dim]."""
        r = f32(rows)
        _check(lib().ora_kv_import(self.h, layer, which, _ptr(r), r.shape[1]))

    def __del__(self):
        try:
            lib().ora_kv_free(self.h)
        except Exception:
            pass


def chacha_block(key, counter: int, stream: int, rounds: int) -> np.ndarray:
    k = np.ascontiguousarray(key, np.uint32)
    out = np.zeros(16, np.uint32)
    _check(lib().ora_chacha_block(_ptr(k), counter, stream, rounds, _ptr(out)))
    return out


class Rng:
    """rand 0.8 StdRng (ChaCha12): seed_from_u64(seed), or from_seed(key)
    with `rounds` rounds when a key is given."""

    def __init__(self, seed: int = 0, rounds: int = 12, key=None):
        h = c_void_p()
        k = None if key is None else np.ascontiguousarray(key, np.uint32)
        _check(lib().ora_rng_create(seed, rounds, None if k is None else _ptr(k), ctypes.byref(h)))
        self.h, self._k = h, k

    def next_u32(self) -> int:
        return int(lib().ora_rng_next_u32(self.h))

    def next_u64(self) -> int:
        return int(lib().ora_rng_next_u64(self.h))

    def gen_f32(self) -> float:
        return float(lib().ora_rng_gen_f32(self.h))

    def gen_f64(self) -> float:
        return float(lib().ora_rng_gen_f64(self.h))

    @staticmethod
    def standard_f32(u: int) -> float:
        """rand's Standard f32 of one u32 (what gen_f32 applies to next_u32)."""
        return float(lib().ora_standard_f32(u))

    @staticmethod
    def standard_f64(u: int) -> float:
        """rand's Standard f64 of one u64."""
        return float(lib().ora_standard_f64(u))

    def key(self) -> np.ndarray:
        k = np.zeros(8, np.uint32)
        lib().ora_rng_key(self.h, _ptr(k))
        return k

    def __del__(self):
        try:
            lib().ora_rng_free(self.h)
        except Exception:
            pass


def softmax_probabilities(logits, temperature: float) -> np.ndarray:
    x = f32(logits)
    out = np.zeros_like(x)
    _check(lib().ora_softmax_probabilities(_ptr(x), x.size, temperature, _ptr(out)))
    return out


def sample_plain(logits, recent, temperature: float, top_k: int, top_p: float, penalty: float, rng: Rng) -> int:
    """apply_repetition_penalty over `recent`, then sample_token with the whole
    SamplerConfig (sampler.rs:47-199)."""
    x = f32(logits)
    r = np.ascontiguousarray(recent, np.int32)
    t = c_int()
    _check(lib().ora_sample_plain(_ptr(x), x.size, _ptr(r) if r.size else None, r.size, temperature, top_k, top_p,
                                  penalty, rng.h, ctypes.byref(t)))
    return t.value


def sample_token(logits, temperature: float, rng: Rng) -> int:
    x = f32(logits)
    t = c_int()
    _check(lib().ora_sample_token(_ptr(x), x.size, temperature, rng.h, ctypes.byref(t)))
    return t.value


def spec_accept(target_logits, draft_logits, draft, temperature: float, rng: Rng):
    """SpeculativeDecoder::step's acceptance (speculative.rs:300-370) with
    sample_correction (speculative.rs:478-513): target rows [k + 1][V],
    draft rows [k][V], draft tokens [k] -> (tokens, accepted)."""
    tl, dl = f32(target_logits), f32(draft_logits)
    d = np.ascontiguousarray(draft, np.int32)
    out = np.zeros(d.size + 1, np.int32)
    prod, acc = c_int(), c_int()
    _check(lib().ora_spec_accept(_ptr(tl), _ptr(dl), tl.shape[1], _ptr(d), d.size, temperature, rng.h, _ptr(out),
                                 ctypes.byref(prod), ctypes.byref(acc)))
    return out[:prod.value].tolist(), acc.value


def sampled_accept(logits, draft, temperature: float, rng: Rng):
    """lookup.rs:359-403 over verify logits [nd + 1][V]: (tokens, accepted)."""
    lg = f32(logits)
    d = np.ascontiguousarray(draft, np.int32)
    out = np.zeros(d.size + 1, np.int32)
    prod, acc = c_int(), c_int()
    _check(lib().ora_sampled_accept(_ptr(lg), lg.shape[1], _ptr(d), d.size, temperature, rng.h, _ptr(out),
                                    ctypes.byref(prod), ctypes.byref(acc)))
    return out[:prod.value].tolist(), acc.value


class LookupDecoder:
    """Oracle counterpart of LookupDecoder (lookup.rs:174-455): greedy
    steps, and exact-sampling steps drawing from an Rng."""

    def __init__(self, model: Model, max_ctx: int):
        h = c_void_p()
        _check(lib().ora_lookup_create(model.h, max_ctx, ctypes.byref(h)))
        self.h = h
        self.model = model

    def prefill(self, prompt) -> int:
        p = np.ascontiguousarray(prompt, np.int32)
        pos = c_int()
        _check(lib().ora_lookup_prefill(self.h, _ptr(p), p.size, ctypes.byref(pos)))
        return pos.value

    def step(self, pos, context, max_draft, min_ngram, max_ngram):
        c = np.ascontiguousarray(context, np.int32)
        out = np.zeros(max_draft + 1, np.int32)
        met = OracleMetrics()
        _check(lib().ora_lookup_step_greedy(self.h, pos, _ptr(c), c.size, max_draft, min_ngram,
                                            max_ngram, _ptr(out), ctypes.byref(met)))
        return out[:met.produced].tolist(), met

    def step_sampled(self, pos, context, max_draft, min_ngram, max_ngram, temperature, rng: Rng):
        c = np.ascontiguousarray(context, np.int32)
        out = np.zeros(max_draft + 1, np.int32)
        met = OracleMetrics()
        _check(lib().ora_lookup_step_sampled(self.h, pos, _ptr(c), c.size, max_draft, min_ngram, max_ngram,
                                             temperature, rng.h, _ptr(out), ctypes.byref(met)))
        return out[:met.produced].tolist(), met

    def kv_filled(self) -> int:
        return lib().ora_lookup_kv_filled(self.h)

    def decode_sample(self, pos: int, token: int, context, temperature: float, top_k: int, top_p: float,
                      penalty: float, rng: "Rng") -> int:
        """The plain sampled step of `rai run` (run.rs:692-735)."""
        c = np.ascontiguousarray(context, np.int32)
        out = np.zeros(1, np.int32)
        _check(lib().ora_lookup_decode_sample(self.h, pos, token, _ptr(c), c.size, temperature, top_k, top_p,
                                              penalty, rng.h, _ptr(out)))
        return int(out[0])

    def decode_one(self, pos: int, token: int) -> int:
        """decode_one (lookup.rs:428-455) with argmax."""
        out = np.zeros(1, np.int32)
        _check(lib().ora_lookup_decode_one(self.h, pos, token, _ptr(out)))
        return int(out[0])

    def import_kv(self, layer: int, which: int, rows: np.ndarray) -> None:
        """Set one layer's K (0) or V (1) cache rows [nkv][npos][head_dim]."""
        r = f32(rows)
        _check(lib().ora_lookup_import_kv(self.h, layer, which, _ptr(r), r.shape[1]))

    def __del__(self):
        try:
            lib().ora_lookup_free(self.h)
        except Exception:
            pass


class SpecDecoder:
    """Oracle SpeculativeDecoder (speculative.rs:61-391); temperature <= 1e-6
    is the greedy variant."""

    def __init__(self, draft: Model, target: Model, max_ctx: int):
        h = c_void_p()
        _check(lib().ora_spec_create(draft.h, target.h, max_ctx, ctypes.byref(h)))
        self.h = h
        self.models = (draft, target)

    def prefill(self, prompt) -> int:
        p = np.ascontiguousarray(prompt, np.int32)
        pos = c_int()
        _check(lib().ora_spec_prefill(self.h, _ptr(p), p.size, ctypes.byref(pos)))
        return pos.value

    def step(self, pos, last, draft_k, temperature, rng):
        out = np.zeros(draft_k + 1, np.int32)
        met = OracleMetrics()
        _check(lib().ora_spec_step(self.h, pos, last, draft_k, temperature, rng.h if rng else None, _ptr(out),
                                   ctypes.byref(met)))
        return out[:met.produced].tolist(), met

    def __del__(self):
        try:
            lib().ora_spec_free(self.h)
        except Exception:
            pass
