"""Numpy restatement of the decode kernel's native expert-block layout.

TEST INFRASTRUCTURE ONLY (imported by tests/ as the checker of
wl_expert_to_native / wl_synth_expert_native). The layout is this build's own
(the reference stores the packed rows as read from its files,
tools/repack_experts_glm.py:46-55); it reorders the same bytes so that every
16-byte load of a GPU wave is one lane of a contiguous 1 KB chunk:

  gu   [I/8 tiles][H/128 k tiles] 1 KB: lane l = (n, g) = (l % 16, l // 16)
       holds row (gate 8T+n if n < 8 else up 8T+n-8), bytes [64kt + 16g, +16)
  gus  [I/8][ceil(H/2048)] 1 KB: lane byte i = scale of that row, k tile
       16c + i, block 4kt + g (0 past the end)
  dn   [I/64 slices][H/32 row pairs] 1 KB: lane holds down row
       32q + n + 16(g >> 1), bytes [32j + 16(g & 1), +16)
  dns  [I/64][ceil(H/512)] 1 KB: lane byte i = scale of that row, pair
       16c + i, block 2j + (g & 1)
"""
import numpy as np


def native_sizes(H, I):
    gu = (I // 8) * (H // 128) * 1024
    gus = (I // 8) * ((H // 128 + 15) // 16) * 1024
    dn = (I // 64) * (H // 32) * 1024
    dns = (I // 64) * ((H // 32 + 15) // 16) * 1024
    return gu, gus, dn, dns


def to_native(parts, H, I):
    """parts = (gw [I,H/2], gs [I,H/32], uw, us, dw [H,I/2], ds [H,I/32]) uint8
    -> the native block (uint8, 1-D)."""
    gw, gs, uw, us, dw, ds = parts
    nkt, nq = H // 128, H // 32
    lane = np.arange(64)
    n, g = lane % 16, lane // 16
    out = []
    # gu
    T = np.arange(I // 8)[:, None, None]
    kt = np.arange(nkt)[None, :, None]
    row = 8 * T + (n & 7)[None, None, :]
    w = np.where((n < 8)[None, None, :, None],
                 gw[row[..., None], 64 * kt[..., None] + 16 * g[None, None, :, None] + np.arange(16)],
                 uw[row[..., None], 64 * kt[..., None] + 16 * g[None, None, :, None] + np.arange(16)])
    out.append(w.reshape(-1))
    # gus
    nc = (nkt + 15) // 16
    T = np.arange(I // 8)[:, None, None, None]
    c = np.arange(nc)[None, :, None, None]
    i = np.arange(16)[None, None, None, :]
    ktv = 16 * c + i
    row = 8 * T + (n & 7)[None, None, :, None]
    col = np.minimum(ktv, nkt - 1) * 4 + g[None, None, :, None]
    s = np.where((n < 8)[None, None, :, None], gs[row, col], us[row, col])
    s = np.where(ktv < nkt, s, 0).astype(np.uint8)
    out.append(s.reshape(-1))
    # dn
    j = np.arange(I // 64)[:, None, None, None]
    q = np.arange(nq)[None, :, None, None]
    row = 32 * q + n[None, None, :, None] + 16 * (g[None, None, :, None] >> 1)
    colb = 32 * j + 16 * (g[None, None, :, None] & 1) + np.arange(16)
    out.append(dw[row, colb].reshape(-1))
    # dns
    ndc = (nq + 15) // 16
    j = np.arange(I // 64)[:, None, None, None]
    c = np.arange(ndc)[None, :, None, None]
    qv = 16 * c + np.arange(16)[None, None, None, :]
    row = 32 * np.minimum(qv, nq - 1) + n[None, None, :, None] + 16 * (g[None, None, :, None] >> 1)
    col = 2 * j + (g[None, None, :, None] & 1)
    s = np.where(qv < nq, ds[row, col], 0).astype(np.uint8)
    out.append(s.reshape(-1))
    return np.concatenate(out).astype(np.uint8)
