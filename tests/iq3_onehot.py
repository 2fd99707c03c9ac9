"""One-hot IQ3_XXS blocks whose dequantized values follow from the block
layout alone (ggml's block_iq3_xxs: f16 d, 64 grid indices, 8 u32 words of
four 7-bit sign indices and a 4-bit scale s; db = d * (0.5 + s) * 0.5).

With d = 1 every value is (2s + 1) / 4 * magnitude, an exact binary
fraction, so each field can be checked on its own against a closed form:
  * scale_blocks: all 16 scale nibbles, signs 0, one grid entry;
  * sign_blocks:  all 128 sign indices (signs: 7 index bits + even parity);
  * grid_blocks:  all 256 grid slots, in order, against IDENT_GRID.
"""
import numpy as np

D_ONE = 0x3C00  # f16 1.0


def _ident_byte(i, k):
    # a distinct-ish magnitude per (entry, byte), always in 1..127
    return 1 + ((i * (2 * k + 1) + 17 * k) % 127)


IDENT_GRID = np.array([sum(_ident_byte(i, k) << (8 * k) for k in range(4)) for i in range(256)],
                      np.uint32)


def mag(grid, i, k):
    return (int(grid[i]) >> (8 * k)) & 0xFF


def _block(qs, aux):
    b = np.zeros(98, np.uint8)
    b[0:2] = np.array([D_ONE], np.uint16).view(np.uint8)
    b[2:66] = np.asarray(qs, np.uint8)
    b[66:98] = np.asarray(aux, np.uint32).view(np.uint8)
    return b


def scale_blocks(grid, entry=1):
    """16 blocks; block s has scale nibble s everywhere, positive signs and
    every index = entry.  Expected y[e] = (2s+1)/4 * mag(entry, e % 4)."""
    blocks, exp = [], []
    for s in range(16):
        blocks.append(_block(np.full(64, entry), np.full(8, s << 28)))
        exp.append([(2 * s + 1) / 4 * mag(grid, entry, e % 4) for e in range(256)])
    return np.stack(blocks), np.array(exp, np.float64)


def sign_blocks(grid, entry=1):
    """4 blocks covering sign indices 0..127 (index 32t + 4ib + l in field l
    of word ib of block t), scale 1.  Returns (blocks, magnitudes, sign
    index per 8-group [4][32])."""
    blocks, mags, idx = [], [], []
    for t in range(4):
        aux, ix = [], []
        for ib in range(8):
            w = 1 << 28
            for l in range(4):
                i = 32 * t + 4 * ib + l
                w |= i << (7 * l)
                ix.append(i)
            aux.append(w)
        blocks.append(_block(np.full(64, entry), aux))
        mags.append([0.75 * mag(grid, entry, e % 4) for e in range(256)])
        idx.append(ix)
    return np.stack(blocks), np.array(mags, np.float64), np.array(idx)


def grid_blocks(grid):
    """4 blocks with indices 64t + p at position p, scale 1, signs 0.
    Expected y[32ib + 8l + j] = 0.75 * mag(64t + 8ib + 2l + j // 4, j % 4)."""
    blocks, exp = [], []
    for t in range(4):
        blocks.append(_block(64 * t + np.arange(64), np.full(8, 1 << 28)))
        e = np.zeros(256)
        for ib in range(8):
            for l in range(4):
                for j in range(8):
                    e[32 * ib + 8 * l + j] = 0.75 * mag(grid, 64 * t + 8 * ib + 2 * l + j // 4, j % 4)
        exp.append(e)
    return np.stack(blocks), np.array(exp, np.float64)


def check_signs(y, mags, idx):
    """y [4][256] from sign_blocks: magnitudes as expected; within each
    8-group the negative elements are the bits of its sign index, bit 7
    being the parity of the other seven (so negatives come in even
    numbers)."""
    y = np.asarray(y, np.float64)
    assert np.array_equal(np.abs(y), mags)
    neg = (y < 0).reshape(4, 32, 8)
    for t in range(4):
        for g in range(32):
            i = int(idx[t][g])
            bits = [(i >> j) & 1 for j in range(7)] + [bin(i).count("1") & 1]
            assert list(neg[t, g].astype(int)) == bits, (t, g, i)
            assert neg[t, g].sum() % 2 == 0
