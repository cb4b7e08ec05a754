"""Test helper: where each element of the GEMM lane layout comes from,
written from the layout's definition (include/tans_amd.h,
tans_fp8_gemm_fused), independently of the encoder's reshapes."""
import numpy as np


def gemm_lane_coords(S, Rp, Nc):
    """(row, column) of element e of every lane: lane
    ((s * (Rp / 16) + g) * 4 + q) * 16 + r holds row 16 g + r; its element e
    is column s Nc + 64 (e // 16) + 16 q + e % 16, or, in a last block of 32
    columns, s Nc + 64 (e // 16) + 8 q + e % 16."""
    K, n = S * Rp * 4, Nc // 4
    lane = np.arange(K)[:, None]
    e = np.arange(n)[None, :]
    r, q = lane % 16, (lane // 16) % 4
    g, s = (lane // 64) % (Rp // 16), lane // (64 * (Rp // 16))
    t = e // 16
    half = (Nc % 64 == 32) & (t == Nc // 64)
    col = s * Nc + 64 * t + np.where(half, 8 * q, 16 * q) + e % 16
    return np.broadcast_to(16 * g + r, (K, n)), col


def matrix_from_lanes(dec, S, Rp, Nc, rows, cols):
    """Scatter decoded lanes [S * Rp * 4, Nc / 4] back to W [rows, cols]."""
    r, c = gemm_lane_coords(S, Rp, Nc)
    full = np.zeros((Rp, S * Nc), dec.dtype)
    full[r, c] = dec
    return full[:rows, :cols]
