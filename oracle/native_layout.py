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
  bgus [ceil(I/256) groups sg][8 waves v][ceil(H/256) steps s] 512 B: lane
       byte 2i + q = scale of the lane's gu row in tile 8(4sg + i) + v, k tile
       2s + q, block 4kt + g (the batched kernels' gate/up scales)
  bdns [ceil(H/512) row blocks rb][8 v][ceil(I/256) steps st] 512 B: lane byte
       2i + h = scale of down row 32q + n + 16(g >> 1), q = 16rb + 2v + h,
       slice 4st + i, block 2j + (g & 1) (the batched kernels' down scales)
(scales past the end of a dimension are 0).
"""
import numpy as np


def native_sizes(H, I):
    gu = (I // 8) * (H // 128) * 1024
    gus = (I // 8) * ((H // 128 + 15) // 16) * 1024
    dn = (I // 64) * (H // 32) * 1024
    dns = (I // 64) * ((H // 32 + 15) // 16) * 1024
    bgus = -(-I // 256) * 8 * -(-H // 256) * 512
    bdns = -(-H // 512) * 8 * -(-I // 256) * 512
    return gu, gus, dn, dns, bgus, bdns


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
    # bgus: [sg][v][s][lane][8]
    S, nstu = I // 64, -(-H // 256)
    sg = np.arange(-(-I // 256))[:, None, None, None, None]
    v = np.arange(8)[None, :, None, None, None]
    st = np.arange(nstu)[None, None, :, None, None]
    bb = np.arange(8)[None, None, None, None, :]
    i, q = bb // 2, bb % 2
    sl = 4 * sg + i
    kt = 2 * st + q
    row = 8 * (8 * np.minimum(sl, S - 1) + v) + (n & 7)[None, None, None, :, None]
    col = 4 * np.minimum(kt, nkt - 1) + g[None, None, None, :, None]
    s = np.where((n < 8)[None, None, None, :, None], gs[row, col], us[row, col])
    s = np.where((sl < S) & (kt < nkt), s, 0).astype(np.uint8)
    out.append(s.reshape(-1))
    # bdns: [rb][v][st][lane][8]
    nj, nstd = I // 64, -(-I // 256)
    rb = np.arange(-(-H // 512))[:, None, None, None, None]
    st = np.arange(nstd)[None, None, :, None, None]
    h = bb % 2
    qq = 16 * rb + 2 * v + h
    sj = 4 * st + i
    row = 32 * np.minimum(qq, nq - 1) + n[None, None, None, :, None] + 16 * (g[None, None, None, :, None] >> 1)
    col = 2 * np.minimum(sj, nj - 1) + (g[None, None, None, :, None] & 1)
    s = np.where((qq < nq) & (sj < nj), ds[row, col], 0).astype(np.uint8)
    out.append(s.reshape(-1))
    return np.concatenate(out).astype(np.uint8)
