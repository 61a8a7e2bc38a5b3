"""Independent float64 numpy restatement used to pin the C oracle.

Written from the ChatNet sources (not from the oracle): block decoders of
DequantQ4_0.cs:28-58, DequantQ4K.cs:37-77 / :218-241 and DequantQ6K.cs:37-88,
and the per-token Llama schedule of LlamaModel.cs:93-346.  Everything here is
vectorised and evaluated in float64, so it shares no accumulation order with
the oracle; agreement to ~1e-5 relative pins the oracle's arithmetic, and a
wrong index, sign or dropped term shows up as an O(1) mismatch.
"""
from __future__ import annotations

import numpy as np


def half(u16: np.ndarray) -> np.ndarray:
    return np.asarray(u16, dtype=np.uint16).view(np.float16).astype(np.float64)


def dequant_q4_0(raw: np.ndarray, n: int) -> np.ndarray:
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 18)
    d = half(b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))
    qs = b[:, 2:]
    q = np.concatenate([qs & 0x0F, qs >> 4], axis=1).astype(np.float64) - 8.0
    return (q * d[:, None]).ravel()[:n]


def q4k_scales(s12: np.ndarray):
    s = np.asarray(s12, dtype=np.int64).reshape(-1, 12)
    sc = np.zeros((s.shape[0], 8), dtype=np.int64)
    m = np.zeros((s.shape[0], 8), dtype=np.int64)
    sc[:, :4] = s[:, 0:4] & 63
    m[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
    m[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, m


def dequant_q4_k(raw: np.ndarray, n: int) -> np.ndarray:
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 144)
    d = half(b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))
    dmin = half(b[:, 2].astype(np.uint16) | (b[:, 3].astype(np.uint16) << 8))
    sc, m = q4k_scales(b[:, 4:16])
    qs = b[:, 16:].reshape(-1, 8, 16)  # sub-block s owns qs[16s:16s+16]
    q = np.concatenate([qs & 0x0F, qs >> 4], axis=2).astype(np.float64)  # [blk, 8, 32]
    val = d[:, None, None] * sc[:, :, None] * q - dmin[:, None, None] * m[:, :, None]
    return val.reshape(-1)[:n]


def dequant_q6_k(raw: np.ndarray, n: int) -> np.ndarray:
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 210)
    d = half(b[:, 208].astype(np.uint16) | (b[:, 209].astype(np.uint16) << 8))
    sc = b[:, 192:208].view(np.int8).astype(np.float64)
    out = np.zeros((b.shape[0], 256))
    for h in range(2):
        ql = b[:, 64 * h: 64 * h + 64].astype(np.int64)
        qh = b[:, 128 + 32 * h: 128 + 32 * h + 32].astype(np.int64)
        l = np.arange(32)
        q1 = (ql[:, l] & 15) | ((qh[:, l] & 3) << 4)
        q2 = (ql[:, l + 32] & 15) | (((qh[:, l] >> 2) & 3) << 4)
        q3 = (ql[:, l] >> 4) | (((qh[:, l] >> 4) & 3) << 4)
        q4 = (ql[:, l + 32] >> 4) | (((qh[:, l] >> 6) & 3) << 4)
        for k, q in enumerate((q1, q2, q3, q4)):
            e = 128 * h + 32 * k + l
            out[:, e] = (q - 32) * sc[:, e // 16]
    return (out * d[:, None]).ravel()[:n]


def dequant_q8_0(raw: np.ndarray, n: int) -> np.ndarray:
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 34)
    d = half(b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))
    q = b[:, 2:].view(np.int8).astype(np.float64)
    return (q * d[:, None]).ravel()[:n]


def dequant_q5_k(raw: np.ndarray, n: int) -> np.ndarray:
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 176)
    d = half(b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8))
    dmin = half(b[:, 2].astype(np.uint16) | (b[:, 3].astype(np.uint16) << 8))
    sc, m = q4k_scales(b[:, 4:16])
    qh = np.unpackbits(b[:, 16:48], axis=1, bitorder="little").reshape(-1, 8, 32)  # bit e of qh
    qs = b[:, 48:].reshape(-1, 8, 16)
    q = np.concatenate([qs & 0x0F, qs >> 4], axis=2).astype(np.float64) + 16.0 * qh
    val = d[:, None, None] * sc[:, :, None] * q - dmin[:, None, None] * m[:, :, None]
    return val.reshape(-1)[:n]


def _h(b, i):
    return half(b[:, i].astype(np.uint16) | (b[:, i + 1].astype(np.uint16) << 8))


def _nibbles32(qs):  # elements 0..15 low nibbles, 16..31 high nibbles (DequantQ4_1.cs:14-16)
    return np.concatenate([qs & 0x0F, qs >> 4], axis=1).astype(np.float64)


def dequant_q4_1(raw: np.ndarray, n: int) -> np.ndarray:  # DequantQ4_1.cs:24-55
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 20)
    return (_nibbles32(b[:, 4:]) * _h(b, 0)[:, None] + _h(b, 2)[:, None]).ravel()[:n]


def _q5(qh4, qs16):  # bit j of the little-endian qh word is element j's fifth bit
    hb = np.unpackbits(qh4, axis=1, bitorder="little").astype(np.float64)  # [blk, 32]
    return _nibbles32(qs16) + 16.0 * hb


def dequant_q5_0(raw: np.ndarray, n: int) -> np.ndarray:  # DequantQ5_0.cs:28-70
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 22)
    return ((_q5(b[:, 2:6], b[:, 6:]) - 16.0) * _h(b, 0)[:, None]).ravel()[:n]


def dequant_q5_1(raw: np.ndarray, n: int) -> np.ndarray:  # DequantQ5_1.cs:30-70
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 24)
    return (_q5(b[:, 4:8], b[:, 8:]) * _h(b, 0)[:, None] + _h(b, 2)[:, None]).ravel()[:n]


def dequant_q2_k(raw: np.ndarray, n: int) -> np.ndarray:  # DequantQ2K.cs:33-86
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 84)
    d, dmin = _h(b, 80), _h(b, 82)
    out = np.zeros((b.shape[0], 256))
    for g in range(2):
        for t in range(4):
            for hh in range(2):
                sb = 8 * g + 2 * t + hh
                q = (b[:, 16 + 32 * g + 16 * hh: 16 + 32 * g + 16 * hh + 16] >> (2 * t)) & 3
                sc, m = (b[:, sb] & 0x0F).astype(np.float64), (b[:, sb] >> 4).astype(np.float64)
                e0 = 128 * g + 32 * t + 16 * hh
                out[:, e0:e0 + 16] = (d * sc)[:, None] * q - (dmin * m)[:, None]
    return out.ravel()[:n]


def q3k_scales(s12: np.ndarray) -> np.ndarray:  # DequantQ3K.cs:122-150
    s = np.asarray(s12, dtype=np.int64).reshape(-1, 12)
    lo = np.concatenate([s[:, 0:8] & 0x0F, s[:, 0:8] >> 4], axis=1)  # sc 0..7 low, 8..15 high nibbles
    hi = np.concatenate([(s[:, 8:12] >> (2 * k)) & 3 for k in range(4)], axis=1)  # sc 4k+i from byte 8+i
    return (lo | (hi << 4)) - 32


def dequant_q3_k(raw: np.ndarray, n: int) -> np.ndarray:  # DequantQ3K.cs:35-70
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 110)
    d = _h(b, 108)
    sc = q3k_scales(b[:, 96:108]).astype(np.float64)
    i = np.arange(256)
    q2 = (b[:, 32 + i // 4] >> (2 * (i % 4))) & 3
    hb = (b[:, i // 8] >> (i % 8)) & 1
    q3 = (q2 | (hb << 2)).astype(np.float64)
    return (d[:, None] * sc[:, i // 16] * (q3 - 4.0)).ravel()[:n]


def dequant_q8_k(raw: np.ndarray, n: int) -> np.ndarray:  # DequantQ8K.cs:26-51
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 292)
    d = b[:, 0:4].copy().view("<f4").astype(np.float64).ravel()
    return (b[:, 4:260].view(np.int8).astype(np.float64) * d[:, None]).ravel()[:n]


# The IQ family as DequantIQ.cs decodes it (bit fields, no codebooks).
IQ4NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float64)


def _bits(b, lo, hi, width):
    """Fields of `width` bits, least significant first, of bytes lo..hi-1 of each block."""
    bits = np.unpackbits(np.ascontiguousarray(b[:, lo:hi]), axis=1, bitorder="little")
    w = bits.reshape(b.shape[0], -1, width)
    return (w * (1 << np.arange(width))).sum(axis=2)


def dequant_iq4_nl(raw: np.ndarray, n: int) -> np.ndarray:  # DequantIQ.cs:46-76
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 18)
    q = _nibbles32(b[:, 2:]).astype(np.int64)
    return (_h(b, 0)[:, None] * IQ4NL[q]).ravel()[:n]


def dequant_iq4_xs(raw: np.ndarray, n: int) -> np.ndarray:  # DequantIQ.cs:139-176
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 136)
    sh = b[:, 2].astype(np.int64) | (b[:, 3].astype(np.int64) << 8)
    sub = np.arange(8)
    sc = ((b[:, 4:12] & 0x3F).astype(np.int64) | (((sh[:, None] >> (2 * sub)) & 3) << 6)) - 32  # bytes 4..11
    qs = b[:, 8:136].reshape(-1, 8, 16)
    q = np.concatenate([qs & 0x0F, qs >> 4], axis=2).astype(np.int64)  # [blk, sub, 32]
    return (_h(b, 0)[:, None, None] * sc[:, :, None] * IQ4NL[q]).ravel()[:n]


def dequant_iq3_s(raw: np.ndarray, n: int) -> np.ndarray:  # DequantIQ.cs:244-290
    flat = np.concatenate([np.asarray(raw, dtype=np.uint8).ravel(), np.zeros(32, np.uint8)])
    nb = (flat.size - 32) // 110
    # each block's window reaches 28 bytes into the next (signs at 98..129, scales at 130..137)
    win = np.stack([flat[110 * k: 110 * k + 138] for k in range(nb)])
    q3 = _bits(win, 2, 66, 2) | (_bits(win, 66, 98, 1) << 2)   # [blk, 256]
    neg = _bits(win, 98, 130, 1)                                # bit j of byte 98+sub: element 8 sub + j
    sc = _bits(win, 130, 138, 2) + 1                            # [blk, 32]: sub-block 4i+k at bits 2k of byte 130+i
    v = _h(win, 0)[:, None] * np.repeat(sc, 8, axis=1) * q3
    return np.where(neg == 1, -v, v).ravel()[:n]


def dequant_iq3_xxs(raw: np.ndarray, n: int) -> np.ndarray:  # DequantIQ.cs:364-399
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 98)
    return (_h(b, 0)[:, None] * (_bits(b, 2, 98, 3) - 4)).ravel()[:n]


def dequant_iq2_xs(raw: np.ndarray, n: int) -> np.ndarray:  # DequantIQ.cs:456-496
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 74)
    sc = _bits(b, 66, 74, 4) - 8            # sub-block 2i low nibble, 2i+1 high nibble of byte 66+i
    return (_h(b, 0)[:, None] * np.repeat(sc, 16, axis=1) * (_bits(b, 2, 66, 2) - 1)).ravel()[:n]


def dequant_iq2_xxs(raw: np.ndarray, n: int) -> np.ndarray:  # DequantIQ.cs:568-598
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 66)
    return (_h(b, 0)[:, None] * (_bits(b, 2, 66, 2) - 1)).ravel()[:n]


def dequant_iq2_s(raw: np.ndarray, n: int) -> np.ndarray:  # DequantIQ.cs:656-696
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 82)
    qh = b[:, 66:82].astype(np.int64)
    v = _h(b, 0)[:, None] * np.repeat((qh & 0x0F) + 1, 16, axis=1) * _bits(b, 2, 66, 2)
    sign = np.zeros((b.shape[0], 16, 16), np.int64)
    sign[:, :, :4] = (qh[:, :, None] >> (4 + np.arange(4))) & 1   # elements 0..3 of each sub-block only
    return np.where(sign.reshape(-1, 256) == 1, -v, v).ravel()[:n]


def _iq1_ternary(b):
    bit = _bits(b, 2, 34, 1)                                    # [blk, 256]: element 8 sub + j
    e = np.arange(256)
    sub, j = e // 8, e % 8
    hbit = (b[:, 34 + sub // 2] >> ((sub % 2) * 4 + j // 2)) & 1
    return np.where(bit == 1, 1, np.where(hbit == 1, -1, 0))


def dequant_iq1_s(raw: np.ndarray, n: int) -> np.ndarray:  # DequantIQ.cs:767-805
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 50)
    return (_h(b, 0)[:, None] * _iq1_ternary(b)).ravel()[:n]


def dequant_iq1_m(raw: np.ndarray, n: int) -> np.ndarray:  # DequantIQ.cs:869-914
    b = np.asarray(raw, dtype=np.uint8).reshape(-1, 56)
    sc = np.where(_bits(b, 50, 54, 1) == 1, 1.0, 0.5)          # sub-block s: bit s%8 of byte 50 + s/8
    return (_h(b, 0)[:, None] * np.repeat(sc, 8, axis=1) * _iq1_ternary(b)).ravel()[:n]


DEQUANT = {2: dequant_q4_0, 8: dequant_q8_0, 12: dequant_q4_k, 13: dequant_q5_k, 14: dequant_q6_k,
           3: dequant_q4_1, 6: dequant_q5_0, 7: dequant_q5_1, 10: dequant_q2_k, 11: dequant_q3_k, 15: dequant_q8_k,
           16: dequant_iq2_xxs, 17: dequant_iq2_xs, 18: dequant_iq3_xxs, 19: dequant_iq1_s, 20: dequant_iq4_nl,
           21: dequant_iq3_s, 22: dequant_iq2_s, 23: dequant_iq4_xs, 29: dequant_iq1_m}


def matrix(t) -> np.ndarray:
    """Dense float64 [rows, cols] of a SynthTensor."""
    cols, rows = int(t.dims[0]), int(t.dims[1]) if len(t.dims) > 1 else 1
    if t.type == 0:
        return t.data.view(np.float32).astype(np.float64).reshape(rows, cols)
    return DEQUANT[t.type](t.data, rows * cols).reshape(rows, cols)


def rmsnorm(x, w, eps):
    return x / np.sqrt(np.mean(x * x) + eps) * w


def rope(v, pos, hd, base):
    v = v.copy().reshape(-1, hd)
    i = np.arange(0, hd, 2)
    theta = pos * base ** (-i / hd)
    c, s = np.cos(theta), np.sin(theta)
    x0, x1 = v[:, 0::2].copy(), v[:, 1::2].copy()
    v[:, 0::2] = x0 * c - x1 * s
    v[:, 1::2] = x0 * s + x1 * c
    return v.ravel()


def rope_neox(v, pos, hd, base):
    """Split-half rotary embedding: element i of a head turns with element
    i + hd/2 by the angle pos * base^(-2i/hd)."""
    v = v.copy().reshape(-1, hd)
    half = hd // 2
    theta = pos * base ** (-2.0 * np.arange(half) / hd)
    c, s = np.cos(theta), np.sin(theta)
    x0, x1 = v[:, :half].copy(), v[:, half:].copy()
    v[:, :half] = x0 * c - x1 * s
    v[:, half:] = x1 * c + x0 * s
    return v.ravel()


class Llama64:
    """float64 LlamaModel (or, for arch 1, QwenModel: q/k/v biases and
    split-half RoPE): same schedule, none of the float32 roundings."""

    def __init__(self, cfg, ck):
        self.cfg = cfg
        self.emb = matrix(ck["token_embd.weight"])
        self.out = matrix(ck["output.weight"]) if "output.weight" in ck else self.emb
        self.out_norm = ck["output_norm.weight"].data.view(np.float32).astype(np.float64)
        self.L = []
        for l in range(cfg.n_layers):
            p = f"blk.{l}."
            self.L.append({k: matrix(ck[p + k + ".weight"]) for k in
                           ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")})
            self.L[-1]["attn_norm"] = ck[p + "attn_norm.weight"].data.view(np.float32).astype(np.float64)
            self.L[-1]["ffn_norm"] = ck[p + "ffn_norm.weight"].data.view(np.float32).astype(np.float64)
            for b in ("attn_q", "attn_k", "attn_v"):
                t = ck.get(p + b + ".bias")
                self.L[-1][b + ".bias"] = np.zeros(0) if t is None else t.data.view(np.float32).astype(np.float64)
        self.kc = np.zeros((cfg.n_layers, cfg.context_length, cfg.kv_dim))
        self.vc = np.zeros_like(self.kc)

    def forward(self, tokens, position):
        c = self.cfg
        hd = c.head_dim
        logits = None
        for t, tok in enumerate(tokens):
            pos = position + t
            x = self.emb[tok].copy()
            for l, W in enumerate(self.L):
                xn = rmsnorm(x, W["attn_norm"], c.rms_norm_eps)
                q, k, v = W["attn_q"] @ xn, W["attn_k"] @ xn, W["attn_v"] @ xn
                if getattr(c, "arch", 0) == 1:
                    if W["attn_q.bias"].size:
                        q, k, v = q + W["attn_q.bias"], k + W["attn_k.bias"], v + W["attn_v.bias"]
                    q, k = rope_neox(q, pos, hd, c.rope_freq_base), rope_neox(k, pos, hd, c.rope_freq_base)
                else:
                    q, k = rope(q, pos, hd, c.rope_freq_base), rope(k, pos, hd, c.rope_freq_base)
                self.kc[l, pos], self.vc[l, pos] = k, v
                att = np.zeros(c.dim)
                for h in range(c.n_heads):
                    kvh = h // c.kv_mul
                    K = self.kc[l, : pos + 1, kvh * hd:(kvh + 1) * hd]
                    V = self.vc[l, : pos + 1, kvh * hd:(kvh + 1) * hd]
                    s = K @ q[h * hd:(h + 1) * hd] / np.sqrt(hd)
                    p = np.exp(s - s.max())
                    p /= p.sum()
                    att[h * hd:(h + 1) * hd] = p @ V
                x = x + W["attn_output"] @ att
                xn = rmsnorm(x, W["ffn_norm"], c.rms_norm_eps)
                g, u = W["ffn_gate"] @ xn, W["ffn_up"] @ xn
                x = x + W["ffn_down"] @ (g / (1 + np.exp(-g)) * u)
            if t == len(tokens) - 1:
                logits = self.out @ rmsnorm(x, self.out_norm, c.rms_norm_eps)
        return logits
