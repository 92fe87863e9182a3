"""K-quant (Q4_K / Q5_K) blocks built from their fields, with ggml's packing rule for the 12-byte scale/min
array (quantize_row_q4_K_ref).  Test data only."""
import numpy as np


def pack_k_scales(sc, mn):
    """ggml quantize_row_q4_K_ref's packing of 8 six-bit (scale, min) pairs into 12 bytes"""
    s = np.zeros(12, np.uint8)
    for j in range(8):
        ls, lm = int(sc[j]), int(mn[j])
        if j < 4:
            s[j] = ls
            s[j + 4] = lm
        else:
            s[j + 4] = (ls & 0xF) | ((lm & 0xF) << 4)
            s[j - 4] |= (ls >> 4) << 6
            s[j] |= (lm >> 4) << 6
    return s


def k_blocks(rng, nblocks, five_bit, d_std=1e-2):
    """random K-quant blocks from their fields, and the fields"""
    out, fields = [], []
    for _ in range(nblocks):
        d = np.float16(rng.normal(0, d_std))
        dmin = np.float16(abs(rng.normal(0, d_std)))
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        q = rng.integers(0, 32 if five_bit else 16, 256)                 # element e -> code
        qs = np.zeros(128, np.uint8)
        qh = np.zeros(32, np.uint8)
        for e in range(256):
            j, l = e // 32, e % 32
            c, h = j // 2, j % 2
            qs[32 * c + l] |= (int(q[e]) & 15) << (4 * h)
            if five_bit:
                qh[l] |= ((int(q[e]) >> 4) & 1) << j
        head = np.concatenate([np.array([d, dmin], np.float16).view(np.uint8), pack_k_scales(sc, mn)])
        out.append(np.concatenate([head, qh, qs]) if five_bit else np.concatenate([head, qs]))
        fields.append((d, dmin, sc, mn, q))
    return np.concatenate(out), fields
