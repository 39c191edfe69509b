"""Readers of the decode kernels' device layouts, written from their documented formulas
(independently of the kernels) for the layout tests."""
import numpy as np


def slot_token(g, j):
    return 16 * (j >> 2) + 4 * g + (j & 3)


def tile_codes(tiles: np.ndarray, bits: int) -> np.ndarray:
    """One 32-token chunk's value tile (512*bits bytes) -> codes[token 0..31][channel 0..127]."""
    words = np.ascontiguousarray(tiles).view(np.uint32)
    out = np.full((32, 128), -1, np.int64)
    slot4, slot8 = [0, 2, 4, 6, 1, 3, 5, 7], [0, 2, 1, 3, 4, 6, 5, 7]
    for w, word in enumerate(words.tolist()):
        if bits == 4:
            blk, l = (w // 256) * 4 + w % 4, (w % 256) // 4
            for k in range(8):
                out[slot_token(l // 16, slot4[k]), 16 * blk + l % 16] = (word >> (4 * k)) & 15
        elif bits == 8:
            blk, l, half = (w // 256) * 2 + (w % 4) // 2, (w % 256) // 4, w % 2
            for k in range(4):
                out[slot_token(l // 16, slot8[4 * half + k]), 16 * blk + l % 16] = (word >> (8 * k)) & 255
        else:
            l, bp = w // 4, w % 4
            for k in range(16):
                blk, slot = 2 * bp + ((k >> 2) & 1), 2 * (k & 3) + (k >> 3)
                out[slot_token(l // 16, slot), 16 * blk + l % 16] = (word >> (2 * k)) & 3
    return out
