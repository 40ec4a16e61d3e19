"""Independent float64 forward of the synthetic int8 decoder.

TEST INFRASTRUCTURE: a numpy restatement of the pre-norm decoder written
from its mathematics, not from the oracle's C code, used to pin the
composition of the oracle's or_decoder_forward (layer wiring, residuals,
RoPE placement, GQA head mapping, the final norm).  Weights are the model's
int8 values times their fp16 group-32 scales; activations are quantized with
QuantizeInt8's rule (absmax/127, round half to even, clamp [-128, 127]) at
the same points as the int8 engine: the normed rows before QKV and gate/up,
every query / key / value head, the attention output row and the SwiGLU
row.  Everything else is float64 (exact softmax, exp, sqrt, cos/sin).

`mistake` plants one composition error in this restatement (never in the
oracle) so a test can show that the comparison detects it.
"""
from __future__ import annotations

import numpy as np

MISTAKES = ("swap_gate_up", "drop_attn_residual", "rope_on_values", "wrong_kv_head", "no_final_norm",
            "rope_off_by_one", "no_scale")


def quantize(x: np.ndarray) -> np.ndarray:
    """QuantizeInt8 over the last axis in float64; returns the dequantized
    values q * scale."""
    peak = np.max(np.abs(x), axis=-1, keepdims=True)
    scale = np.where(peak > 0, peak / 127.0, 1.0)
    q = np.clip(np.rint(x / scale), -128, 127)
    return q * scale


def dequant(w: np.ndarray, s: np.ndarray) -> np.ndarray:
    hs = s.view(np.float16).astype(np.float64)
    return w.astype(np.float64) * np.repeat(hs, 32, axis=1)


def rmsnorm(x, gain, eps):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * gain.astype(np.float64)


def rope(v: np.ndarray, pos: int, theta: float) -> np.ndarray:
    """Rotate-half rotary position of one 64-wide head at position pos."""
    half = v.shape[-1] // 2
    ang = pos * theta ** (-2.0 * np.arange(half) / v.shape[-1])
    c, s = np.cos(ang), np.sin(ang)
    x0, x1 = v[..., :half], v[..., half:]
    return np.concatenate([x0 * c - x1 * s, x1 * c + x0 * s], axis=-1)


class Float64Decoder:
    """Holds a float64 KV cache per slot: keys / values as their quantized
    values (q * scale), as the int8 cache stores them."""

    def __init__(self, model: dict, slots: int, mistake: str | None = None):
        assert mistake is None or mistake in MISTAKES, mistake
        self.m = model
        self.D = model["dims"]
        self.mistake = mistake
        D = self.D
        self.W = []
        for lw in model["layers"]:
            self.W.append({n: dequant(lw["w" + n], lw["s" + n]) for n in ("qkv", "o", "gu", "d")})
        self.Wlm = dequant(model["wlm"], model["slm"])
        self.cache = [[{} for _ in range(slots)] for _ in range(D["layers"])]

    def forward(self, tokens, slots, positions) -> np.ndarray:
        D, mk = self.D, self.mistake
        d, H, KV, hd, F = D["d"], D["heads"], D["kv_heads"], D["head_dim"], D["ffn"]
        group = H // KV
        x = self.m["embedding"][np.asarray(tokens)].astype(np.float64)
        rows = len(tokens)
        for l, lw in enumerate(self.m["layers"]):
            W = self.W[l]
            h = quantize(rmsnorm(x, lw["attn_norm"], D["eps"]))
            qkv = h @ W["qkv"].T
            att = np.zeros((rows, H * hd))
            for r in range(rows):
                p, sl = int(positions[r]), int(slots[r])
                rp = p + 1 if mk == "rope_off_by_one" else p
                q = qkv[r, :H * hd].reshape(H, hd)
                k = qkv[r, H * hd:(H + KV) * hd].reshape(KV, hd)
                v = qkv[r, (H + KV) * hd:].reshape(KV, hd)
                q = quantize(rope(q, rp, D["theta"]))
                k = quantize(rope(k, rp, D["theta"]))
                v = quantize(rope(v, rp, D["theta"]) if mk == "rope_on_values" else v)
                self.cache[l][sl][p] = (k, v)
            for r in range(rows):  # attention after every row of the forward wrote its position
                p, sl = int(positions[r]), int(slots[r])
                q = quantize(rope(qkv[r, :H * hd].reshape(H, hd), p + 1 if mk == "rope_off_by_one" else p,
                                  D["theta"]))
                ks = np.stack([self.cache[l][sl][s][0] for s in range(p + 1)])  # [pos][KV][hd]
                vs = np.stack([self.cache[l][sl][s][1] for s in range(p + 1)])
                for hh in range(H):
                    kvh = (hh + 1) % KV if mk == "wrong_kv_head" else hh // group
                    sc = ks[:, kvh, :] @ q[hh]
                    if mk != "no_scale":
                        sc = sc / np.sqrt(hd)
                    e = np.exp(sc - sc.max())
                    att[r, hh * hd:(hh + 1) * hd] = (e / e.sum()) @ vs[:, kvh, :]
            delta = quantize(att) @ W["o"].T
            x = delta if mk == "drop_attn_residual" else x + delta
            h = quantize(rmsnorm(x, lw["ffn_norm"], D["eps"]))
            gu = h @ W["gu"].T
            g, u = (gu[:, F:], gu[:, :F]) if mk == "swap_gate_up" else (gu[:, :F], gu[:, F:])
            a = quantize(g / (1.0 + np.exp(-g)) * u)
            x = x + a @ W["d"].T
        h = x if mk == "no_final_norm" else rmsnorm(x, self.m["final_norm"], D["eps"])
        return quantize(h) @ self.Wlm.T
