"""A float64 "textbook" Llama/OLMoE forward pass over a .raimodel file.

Test infrastructure: an independent statement of the model composition the
reference implements in rai-infer/src/model.rs:692-1033 (forward_batch and
hidden_to_logits_batch), written from the model's definition rather than from
the AVX2 code, used to pin the oracle's layer composition (GQA head mapping,
RoPE pairing, residual and norm placement, MoE routing and accumulation).

Everything is float64 except the two places where the reference's arithmetic
is itself part of the model's definition and is emulated per that definition:
  * activations entering every W4A8 projection are quantized per group to
    int8 (gemm.rs:280-374: scale absmax/127, round to nearest even, clamp),
    and the zero-point term uses the raw input sum (gemm.rs:528-537):
        y_r = sum_g ws_rg * as_g * sum_c code_rc * q_c + z_rg * sum_c x_c;
    the tied 8-bit head quantizes to +-63 the same way (gemm.rs:924-965);
  * the 8-aligned bodies of the attention softmax and of SiLU use
    Schraudolph's exponential (layers.rs:855-876, 1317-1331), whose f32
    steps are reproduced in numpy float32; tails use the exact exponential.
"""
from __future__ import annotations

import struct

import numpy as np


def schraudolph(d) -> np.ndarray:
    """layers.rs:855-876 per lane: f32(f32(12102203 * d) + 1064866816),
    clamped to [0, 2139095040], rounded to nearest even, read as f32 bits."""
    d = np.asarray(d, np.float32)
    t = np.float32(12102203.0) * d + np.float32(1064866816.0)
    t = np.minimum(t, np.float32(2139095040.0))
    t = np.maximum(t, np.float32(0.0))
    return np.rint(t).astype(np.int32).view(np.float32).astype(np.float64)


class Linear:
    def __init__(self, data: bytes, off: int, gs: int):
        rows, cols = struct.unpack_from("<II", data, off)
        groups = -(-cols // gs)
        par = np.frombuffer(data, np.float16, rows * groups * 2, off + 8).reshape(rows, groups, 2)
        nib = np.frombuffer(data, np.uint8, rows * cols // 2, off + 8 + rows * groups * 4)
        codes = np.empty(rows * cols, np.float64)
        codes[0::2] = nib & 15   # low nibble = even column
        codes[1::2] = nib >> 4
        self.rows, self.cols, self.gs, self.groups = rows, cols, gs, groups
        self.codes = codes.reshape(rows, cols)
        self.scale = par[:, :, 0].astype(np.float64)
        self.zero = par[:, :, 1].astype(np.float64)
        self.end = off + 8 + rows * groups * 4 + rows * cols // 2

    def __call__(self, x: np.ndarray) -> np.ndarray:
        """W4A8 product of one row x [cols] (float64 emulation)."""
        gs, G = self.gs, self.groups
        pad = G * gs - self.cols
        xp = np.concatenate([x, np.zeros(pad)]).reshape(G, gs)
        absmax = np.abs(xp).max(axis=1)
        s = np.where(absmax > 1e-10, absmax / 127.0, 1.0)
        q = np.clip(np.rint(xp / s[:, None]), -128, 127)
        cp = np.concatenate([self.codes, np.zeros((self.rows, pad))], axis=1).reshape(self.rows, G, gs)
        S = np.einsum("rgc,gc->rg", cp, q)
        return (self.scale * s[None, :] * S).sum(axis=1) + (self.zero * xp.sum(axis=1)[None, :]).sum(axis=1)


class TextbookModel:
    def __init__(self, data: bytes, mistake: str | None = None):
        """`mistake` plants one deliberate error in the composition, so that a
        test can show the comparison notices it: "gqa" (kv head qh % nkv
        instead of qh // (nh / nkv)), "rope_sign" (x0 c + x1 s), "rope_pairs"
        (adjacent pairs instead of the half split), "no_attn_residual",
        "norm_swap" (the two layer norms exchanged), "scale" (1 / head_dim
        instead of 1 / sqrt(head_dim)), "topk_ties" (MoE ties to the highest
        index) or "moe_renorm" (renormalised top-k weights)."""
        self.mistake = mistake
        d = bytes(data)
        assert d[:4] == b"RAIM"
        ver = struct.unpack_from("<I", d, 4)[0]
        (self.H, self.L, self.nh, self.nkv, self.hd, self.F, self.V,
         self.max_ctx) = struct.unpack_from("<8I", d, 8)
        self.theta, self.eps = struct.unpack_from("<ff", d, 40)
        self.gs, self.egs = d[49], d[51]
        nsec = struct.unpack_from("<I", d, 52)[0]
        hsz = 64 if ver == 1 else 128
        secs = [struct.unpack_from("<QQ", d, hsz + 16 * i) for i in range(nsec)]
        self.E = self.topk = 0
        self.norm_topk = False
        self.attn_scale = 1.0 / np.sqrt(self.hd)
        if ver == 2:
            asc = struct.unpack_from("<f", d, 96)[0]
            if asc != 0.0:
                self.attn_scale = asc
            self.E = struct.unpack_from("<H", d, 105)[0]
            self.topk = d[107]
            self.norm_topk = bool(d[108] & 1)
        if mistake == "gqa":
            self.gqa_map = lambda qh, nh, nkv: qh % nkv
        else:
            self.gqa_map = lambda qh, nh, nkv: qh // (nh // nkv)
        if mistake == "scale":
            self.attn_scale = 1.0 / self.hd
        if mistake == "moe_renorm":
            self.norm_topk = not self.norm_topk
        H, V, egs = self.H, self.V, self.egs
        eg = -(-H // egs)
        off = secs[0][0]
        ep = np.frombuffer(d, np.float16, V * eg * 2, off).reshape(V, eg, 2).astype(np.float64)
        ec = np.frombuffer(d, np.uint8, V * H, off + V * eg * 4).reshape(V, H).astype(np.float64)
        self.emb_codes, self.emb_scale, self.emb_zero = ec, ep[:, :, 0], ep[:, :, 1]
        self.layers = []
        for li in range(self.L):
            off = secs[1 + li][0]
            lins = []
            for _ in range(7):
                lin = Linear(d, off, self.gs)
                lins.append(lin)
                off = lin.end
            layer = {"lin": lins}
            if self.E:
                layer["router"] = np.frombuffer(d, np.float32, self.E * H, off).reshape(self.E, H).astype(np.float64)
                off += self.E * H * 4
                experts = [lins[4:7]]
                for _ in range(self.E - 1):
                    ex = []
                    for _ in range(3):
                        lin = Linear(d, off, self.gs)
                        ex.append(lin)
                        off = lin.end
                    experts.append(ex)
                layer["experts"] = experts
            norms = [np.frombuffer(d, np.float32, H, off + 4 * H * i).astype(np.float64) for i in (0, 1)]
            if mistake == "norm_swap":
                norms.reverse()
            layer["in_norm"], layer["post_norm"] = norms
            self.layers.append(layer)
        self.final_norm = np.frombuffer(d, np.float32, H, secs[self.L + 1][0]).astype(np.float64)
        self.lm_head = Linear(d, secs[self.L + 2][0], self.gs) if nsec == self.L + 3 else None

    def embed(self, token: int) -> np.ndarray:
        g = np.arange(self.H) // self.egs
        return self.emb_codes[token] * self.emb_scale[token, g] + self.emb_zero[token, g]

    def _norm(self, x, w):
        return x / np.sqrt(np.mean(x * x) + np.float64(self.eps)) * w

    def _rope(self, x, nheads, pos):
        half = self.hd // 2
        inv = self.theta ** (-2.0 * np.arange(half) / self.hd)
        c, s = np.cos(pos * inv), np.sin(pos * inv)
        x = x.reshape(nheads, self.hd).copy()
        i0, i1 = np.arange(half), np.arange(half) + half  # (i, i + hd/2) pairs
        if self.mistake == "rope_pairs":
            i0, i1 = 2 * np.arange(half), 2 * np.arange(half) + 1
        x0, x1 = x[:, i0].copy(), x[:, i1].copy()
        sign = -1.0 if self.mistake == "rope_sign" else 1.0
        x[:, i0] = x0 * c - sign * x1 * s
        x[:, i1] = x1 * c + sign * x0 * s
        return x.reshape(-1)

    def _attend(self, q, ks, vs):
        n = ks.shape[0]
        sc = (ks @ q) * self.attn_scale
        d = sc - sc.max()
        n8 = 8 * (n // 8)
        e = np.concatenate([schraudolph(d[:n8]), np.exp(d[n8:])])
        return (e / e.sum()) @ vs

    def _silu_mul(self, g, u):
        n8 = 8 * (g.size // 8)
        e = np.concatenate([schraudolph(-g[:n8]), np.exp(-g[n8:])])
        return g / (1.0 + e) * u

    def _mlp(self, layer, x):
        if not self.E:
            gate, up, down = layer["lin"][4:7]
            return down(self._silu_mul(gate(x), up(x)))
        logits = layer["router"] @ x
        p = np.exp(logits - logits.max())
        p /= p.sum()
        tie = 1 if self.mistake == "topk_ties" else -1
        order = sorted(range(self.E), key=lambda e: (-p[e], -tie * e))[:self.topk]
        w = p[order]
        if self.norm_topk:
            w = w / w.sum()
        out = np.zeros(self.H)
        for e, we in zip(order, w):
            gate, up, down = layer["experts"][e]
            out += we * down(self._silu_mul(gate(x), up(x)))
        return out

    def forward(self, tokens) -> np.ndarray:
        """Logits [len(tokens), V] of a causal pass over positions 0.."""
        return self.logits(self.hidden(tokens))

    def hidden(self, tokens) -> np.ndarray:
        """Hidden states [len(tokens), H] after the last layer."""
        H, nh, nkv, hd = self.H, self.nh, self.nkv, self.hd
        hs = [self.embed(t) for t in tokens]
        T = len(tokens)
        for layer in self.layers:
            q_, k_, v_, o_ = layer["lin"][:4]
            K = np.zeros((nkv, T, hd))
            Vc = np.zeros((nkv, T, hd))
            qs = []
            for p in range(T):
                n = self._norm(hs[p], layer["in_norm"])
                qs.append(self._rope(q_(n), nh, p).reshape(nh, hd))
                K[:, p] = self._rope(k_(n), nkv, p).reshape(nkv, hd)
                Vc[:, p] = v_(n).reshape(nkv, hd)
            for p in range(T):
                att = np.concatenate([self._attend(qs[p][qh], K[self.gqa_map(qh, nh, nkv), :p + 1],
                                                   Vc[self.gqa_map(qh, nh, nkv), :p + 1])
                                      for qh in range(nh)])
                h = (0.0 if self.mistake == "no_attn_residual" else hs[p]) + o_(att)
                hs[p] = h + self._mlp(layer, self._norm(h, layer["post_norm"]))
        return np.stack(hs)

    def logits(self, hs) -> np.ndarray:
        out = []
        for h in hs:
            n = self._norm(h, self.final_norm)
            if self.lm_head is not None:
                out.append(self.lm_head(n))
            else:
                out.append(self._tied_head(n))
        return np.stack(out)

    def _tied_head(self, x):
        egs, G = self.egs, -(-self.H // self.egs)
        pad = G * egs - self.H
        xp = np.concatenate([x, np.zeros(pad)]).reshape(G, egs)
        absmax = np.abs(xp).max(axis=1)
        s = np.where(absmax > 1e-10, absmax / 63.0, 1.0)
        q = np.clip(np.rint(xp / s[:, None]), -63, 63)
        cp = np.concatenate([self.emb_codes, np.zeros((self.V, pad))], axis=1).reshape(self.V, G, egs)
        S = np.einsum("vgc,gc->vg", cp, q)
        return (self.emb_scale * s[None, :] * S).sum(axis=1) + (self.emb_zero * xp.sum(axis=1)[None, :]).sum(axis=1)
