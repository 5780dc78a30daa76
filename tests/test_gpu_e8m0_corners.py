"""E8M0 corner scales through the hot kernels (GPU; run with -m gpu).

GLM-shape expert blocks (and the shared expert) with planted rows whose
scales are the E8M0 corners, so that those values dominate the rows they are
in, run through the decode kernel (both schedules) and the batched layer (one
pass of more than 32 tokens per expert), against the oracle's dequant
(tools/glm_mxfp4_numpy.py:17-26, exact ldexp; src/glm_kernels.cuh:53-61):

  gate/up rows (routed SwiGLU values, checked through the mid tap)
    A  gate row at E8M0 1 (weights 2^-127 .. 1.5 x 2^-124: bf16 subnormals
       included), up row normal: mid ~ 1e-35
    B  gate row at E8M0 200 (2^73), up row at E8M0 54 (2^-73): mid ~ 1e4
    C  gate row with one E8M0-254 block holding a single 0.5 (2^126) at a
       column whose normalised input stays below 1.5, up row at E8M0 1
    G  gate and up rows at E8M0 116 (small SwiGLU values, |mid| < 1)
  down rows (layer output, the shared expert's row zeroed)
    D  down row at E8M0 200: output ~ 1e23
    E  down row at E8M0 1: output ~ 1e-36
    F  down row with one E8M0-254 block holding a single 0.5 (2^126) at
       expert k's G column: output ~ 1e35

A planted value is one dot product (or a SwiGLU of two, or a sum of down
products), so it is held to the reference's own matvec bar: within 1e-5 of
its term magnitudes (term-relative, src/test_glm_mxfp4.cu:186-191), carried
through silu(g) * u and the down projection to first order; every other
output row to the usual 1e-5 rel_to_scale over those rows. Experts are chosen
by the router bias (+10 on the planted 8), so the routing is fixed; ids are
compared exactly. The overflow
case (E8M0 254 with |e2m1| >= 2) is pinned in tests/test_gpu_mxfp4_edges.py.
"""
import numpy as np
import pytest

from oracle import moe_oracle as O
from oracle import synth
from windlass_amd import hip as H_
from windlass_amd import moe, synthdata

pytestmark = pytest.mark.gpu
TOL = 1e-5
GLM = dict(hidden=6144, moe_inter=2048, n_routed_experts=256, n_experts_per_tok=8, n_shared=1,
           routed_scaling=2.5, rms_eps=1e-5)
SEED = 23
PLANTED = [3, 41, 77, 100, 133, 180, 201, 250]
ROWS_A = [10, 1030]
ROWS_B = [300, 1800]
ROWS_C = [600]
ROWS_G = [900]
ROWS_D = [11, 3000]
ROWS_E = [500, 4096]
ROWS_F = [2000, 6143]
T_BATCH = 40


def _hidden(n):
    H = GLM["hidden"]
    return np.stack([synthdata.hidden_state(H, 600 + t) for t in range(n)]).astype(np.float32)


def _single(row_nib, row_sc, col, sc):
    """The row's block holding `col` at scale `sc` with a single 0.5 (code 1)
    at `col`, every other value of the block zero."""
    b = col // 32
    row_nib[16 * b:16 * b + 16] = 0
    row_nib[col // 2] = 0x01 if col % 2 == 0 else 0x10
    row_sc[b] = sc


def _plant_gate_up(gw, gs, uw, us, rows_shift, col_c):
    for r in ROWS_A:
        gs[r + rows_shift] = 1
    for r in ROWS_B:
        gs[r + rows_shift] = 200
        us[r + rows_shift] = 54
    for r in ROWS_C:
        _single(gw[r + rows_shift], gs[r + rows_shift], col_c, 254)
        us[r + rows_shift] = 1
    for r in ROWS_G:
        gs[r + rows_shift] = 116
        us[r + rows_shift] = 116


def _pack(parts):
    return np.concatenate([p.reshape(-1) for p in parts]).astype(np.uint8)


@pytest.fixture(scope="module")
def corners(gpu):
    c = GLM
    H, I, E, K = c["hidden"], c["moe_inter"], c["n_routed_experts"], c["n_experts_per_tok"]
    hs = _hidden(3 + T_BATCH)
    xn = O.rms_norm(hs, None, c["rms_eps"])
    col_c = int(np.argmin(np.abs(xn).max(axis=0)))  # the input column that stays smallest
    assert np.abs(xn[:, col_c]).max() < 1.5  # 2^126 x 1.5 stays finite
    blocks = {}
    for k, e in enumerate(PLANTED):
        gw, gs, uw, us, dw, ds = [a.copy() for a in synth.expert_block(H, I, SEED, 0, e)]
        _plant_gate_up(gw, gs, uw, us, k, col_c)
        for r in ROWS_D:
            ds[r] = 200
        for r in ROWS_E:
            ds[r] = 1
        for r in ROWS_F:  # 2^126 x expert k's G value: far above the row's other terms, below overflow
            _single(dw[r], ds[r], ROWS_G[0] + k, 254)
        blocks[e] = [gw, gs, uw, us, dw, ds]
        g_mid = O.swiglu_mid(xn, O.dequant(gw[ROWS_G[0] + k][None], gs[ROWS_G[0] + k][None]),
                             O.dequant(uw[ROWS_G[0] + k][None], us[ROWS_G[0] + k][None]))
        assert np.abs(g_mid).max() < 1.0 and np.abs(g_mid).min() > 0
    dense = synthdata.dense_layer(H, E, I, SEED, 0)
    off = np.zeros(E, np.float32)
    off[PLANTED] = 10.0
    dense["bias"] = (dense["bias"] + off).astype(np.float32)
    # bf16 shared expert: its rows of the planted outputs zeroed
    sd = dense["sh_down"].copy()
    sd[ROWS_D + ROWS_E + ROWS_F] = 0
    dense["sh_down"] = sd
    dense["shared_block"] = np.concatenate([dense["sh_gate"].reshape(-1), dense["sh_up"].reshape(-1), sd.reshape(-1)])
    # MXFP4 shared expert: the same planted gate/up kinds (rows shifted by 8),
    # its rows of the planted outputs zeroed
    sh4 = [a.copy() for a in synth.expert_block(H, I, SEED, 0, 0xFFFF)]
    _plant_gate_up(sh4[0], sh4[1], sh4[2], sh4[3], 8, col_c)
    sh4[4][ROWS_D + ROWS_E + ROWS_F] = 0

    cfg = moe.make_config(n_layers=1)
    ctx = moe.Context(cfg)
    ctx.slot_pool_create(K + 1)
    lay = moe.expert_layout(cfg)
    staging = H_.DeviceBuffer(lay.total)
    for k, e in enumerate(PLANTED):
        staging.upload(_pack(blocks[e]))
        moe.expert_to_native(cfg, staging.ptr, ctx.slot_pool_ptr(k))
        H_.synchronize()
        ctx.slot_bind(0, e, ctx.slot_pool_ptr(k))
    moe.synth_expert_native(cfg, SEED, 0, 0, ctx.slot_pool_ptr(K))  # never routed
    for e in range(E):
        if e not in blocks:
            ctx.slot_bind(0, e, ctx.slot_pool_ptr(K))
    bufs = {"rw": H_.DeviceBuffer.from_array(dense["router_w"]), "b": H_.DeviceBuffer.from_array(dense["bias"]),
            "bf16": H_.DeviceBuffer.from_array(dense["shared_block"]), "mx": H_.DeviceBuffer.from_array(_pack(sh4))}
    H_.synchronize()

    class Src:
        def __init__(self):
            self.cache = {}

        def get(self, layer, e):
            if e not in self.cache:
                b = blocks[e]
                self.cache[e] = (O.dequant(b[0], b[1]), O.dequant(b[2], b[3]), O.dequant(b[4], b[5]))
            return self.cache[e]

    shared4 = (O.dequant(sh4[0], sh4[1]), O.dequant(sh4[2], sh4[3]), O.dequant(sh4[4], sh4[5]))
    yield {"ctx": ctx, "bufs": bufs, "dense": dense, "src": Src(), "hs": hs, "shared4": shared4}
    ctx.close()


def _bind_shared(f, shared):
    b = f["bufs"]
    if shared == "bf16":
        f["ctx"].set_layer(0, b["rw"].ptr, b["b"].ptr, None, b["bf16"].ptr, moe.SHARED_BF16)
        return None
    f["ctx"].set_layer(0, b["rw"].ptr, b["b"].ptr, None, b["mx"].ptr, moe.SHARED_MXFP4)
    return f["shared4"]


def _silu_and_slope(g):
    """silu(g) and its derivative in f64, finite for any g."""
    sg = 0.5 * (1.0 + np.tanh(0.5 * g))
    return g * sg, sg + g * sg * (1.0 - sg)


def _mid_scales(f, ids, X):
    """Per slot k and token t: the SwiGLU values' term scales S[t, k, :]
    (f64), the first-order bound of |d mid| when the gate and up dot products
    are each off by their term magnitudes sum_c |w_c x_c|: a term-relative
    bar of 1e-5 (the reference's matvec bar, src/test_glm_mxfp4.cu:186-191)
    carried through silu(g) * u. Also the f64 SwiGLU values."""
    X64 = np.atleast_2d(X).astype(np.float64)
    S, M = [], []
    for e in ids:
        G, U, _ = f["src"].get(0, int(e))
        g = X64 @ G.T.astype(np.float64)
        u = X64 @ U.T.astype(np.float64)
        tg = np.abs(X64) @ np.abs(G.T).astype(np.float64)
        tu = np.abs(X64) @ np.abs(U.T).astype(np.float64)
        sg, ds = _silu_and_slope(g)
        S.append(np.abs(ds) * tg * np.abs(u) + np.abs(sg) * tu)
        M.append(sg * u)
    return np.stack(S, axis=1), np.stack(M, axis=1)


def _check_rows(f, ids, wts, S, M, ref, got, what):
    """Planted output rows: |got - ref| within 1e-5 of the row's term scale
    sum_k |w_k| sum_c |D_k[r, c]| (|mid_k[c]| + S_k[c]) (the down products'
    terms and the SwiGLU values' own bound); every other row: rel_to_scale
    over those rows (the vector bar)."""
    planted = ROWS_D + ROWS_E + ROWS_F
    ts = np.zeros(len(planted))
    for k, e in enumerate(ids):
        D = f["src"].get(0, int(e))[2][planted].astype(np.float64)
        ts += abs(float(wts[k])) * (np.abs(D) @ (np.abs(M[k]) + S[k]))
    err = np.abs(got[planted].astype(np.float64) - ref[planted])
    assert np.all(err <= TOL * ts), (what, planted, err / ts, ref[planted], got[planted])
    rest = np.setdiff1d(np.arange(ref.shape[0]), planted)
    r = O.rel_to_scale(ref[rest], got[rest])
    assert r < TOL, (what, "rest", r)
    return {n: float(np.abs(ref[rows]).max()) for n, rows in (("D", ROWS_D), ("E", ROWS_E), ("F", ROWS_F))}


@pytest.mark.parametrize("shared", ["bf16", "mxfp4"])
def test_corner_scales_through_decode(corners, shared):
    f = corners
    ctx, c = f["ctx"], GLM
    H, I, K = c["hidden"], c["moe_inter"], c["n_experts_per_tok"]
    sh = _bind_shared(f, shared)
    dh, dout = H_.DeviceBuffer(4 * H), H_.DeviceBuffer(4 * H)
    outs = {}
    for sched in (moe.SCHED_FUSED, moe.SCHED_PHASED):
        ctx.set_schedule(sched)
        for t in range(3):
            h = f["hs"][t]
            dh.upload(h)
            ctx.run_moe(0, dh.ptr, dout.ptr)
            ctx.check_error()
            out = dout.download(np.float32)
            ref = O.moe_layer(h, f["dense"], f["src"], 0, c, shared_f32=sh)
            tp = ctx.taps()
            ids = H_.download_ptr(tp["topk_idx"], np.int32, K)
            assert sorted(ids.tolist()) == sorted(PLANTED)
            assert np.array_equal(ids, ref["topk_idx"])
            mid = H_.download_ptr(tp["mid"], np.float32, K * I).reshape(K, I)
            S, M = _mid_scales(f, ids, O.rms_norm(h, None, c["rms_eps"]))
            S, M = S[0], M[0]
            for k, e in enumerate(ids):
                p = PLANTED.index(int(e))  # the expert's planted rows are shifted by its index
                for name, rows in (("A", ROWS_A), ("B", ROWS_B), ("C", ROWS_C), ("G", ROWS_G)):
                    rr = [r + p for r in rows]
                    err = np.abs(mid[k][rr].astype(np.float64) - ref["mid"][k][rr])
                    assert np.all(err <= TOL * S[k][rr]), (shared, sched, t, int(e), name, err, S[k][rr])
            if shared == "mxfp4":
                got_sh = H_.download_ptr(tp["shared"], np.float32, H)
                assert O.rel_to_scale(ref["shared"], got_sh) < TOL
            mags = _check_rows(f, ids, ref["topk_w"], S, M, ref["out"], out, (shared, sched, t))
            outs[(sched, t)] = out
        print(f"decode ({shared} shared), schedule {sched}: planted row magnitudes {mags}", flush=True)
    for t in range(3):
        assert np.array_equal(outs[(moe.SCHED_FUSED, t)].view(np.uint32), outs[(moe.SCHED_PHASED, t)].view(np.uint32))
    ctx.set_schedule(moe.SCHED_FUSED)


@pytest.mark.parametrize("shared", ["bf16", "mxfp4"])
def test_corner_scales_through_batched(corners, shared):
    f = corners
    ctx, c = f["ctx"], GLM
    H = c["hidden"]
    sh = _bind_shared(f, shared)
    hs = f["hs"][3:3 + T_BATCH]
    d_in = H_.DeviceBuffer.from_array(hs)
    d_out = H_.DeviceBuffer(4 * H * T_BATCH)
    ctx.run_moe_batched(0, T_BATCH, d_in.ptr, None, d_out.ptr)
    ctx.check_error()
    counts = ctx.batched_counts()
    assert counts.max() == T_BATCH  # one pass of 32 tokens and one of 8 per planted expert
    out = d_out.download(np.float32).reshape(T_BATCH, H)
    ids = None
    for t in range(T_BATCH):
        ref = O.moe_layer(hs[t], f["dense"], f["src"], 0, c, shared_f32=sh)
        if ids is None or not np.array_equal(ids, ref["topk_idx"]):
            ids = ref["topk_idx"]
        S, M = _mid_scales(f, ids, O.rms_norm(hs[t], None, c["rms_eps"]))
        _check_rows(f, ids, ref["topk_w"], S[0], M[0], ref["out"], out[t], (shared, "batched", t))
    print(f"batched ({shared} shared): {T_BATCH} tokens, planted rows within {TOL}", flush=True)


@pytest.mark.parametrize("shared", ["bf16", "mxfp4"])
def test_corner_scales_through_batched_wide_passes(corners, shared):
    """1024 tokens, all routed to the planted experts: every planted expert
    (and the shared expert) runs in the batched kernels' wide passes (tokens
    split evenly over passes of at most 48, the shared expert in passes of
    64). Twelve tokens spread over the passes are held to the corner bars
    against the oracle; every token's other output rows to 1e-5 against the
    decode kernel (the planted down rows D, E, F scale a SwiGLU value by up to
    2^126, so two implementations that each meet its term-relative bar can
    differ there by more than 1e-5 of the row scale)."""
    f = corners
    ctx, c = f["ctx"], GLM
    H, T = c["hidden"], 1024
    sh = _bind_shared(f, shared)
    hs = _hidden(T)
    d_in = H_.DeviceBuffer.from_array(hs)
    d_out = H_.DeviceBuffer(4 * H * T)
    ctx.run_moe_batched(0, T, d_in.ptr, None, d_out.ptr)
    ctx.check_error()
    counts = ctx.batched_counts()
    assert sorted(np.nonzero(counts)[0].tolist())[:8] == PLANTED and counts.max() == T
    out = d_out.download(np.float32).reshape(T, H)
    for t in (0, 1, 21, 22, 47, 48, 300, 511, 512, 700, 1000, 1023):
        ref = O.moe_layer(hs[t], f["dense"], f["src"], 0, c, shared_f32=sh)
        S, M = _mid_scales(f, ref["topk_idx"], O.rms_norm(hs[t], None, c["rms_eps"]))
        _check_rows(f, ref["topk_idx"], ref["topk_w"], S[0], M[0], ref["out"], out[t], (shared, "wide", t))
    d_h, d_o = H_.DeviceBuffer(4 * H), H_.DeviceBuffer(4 * H)
    rest = np.setdiff1d(np.arange(H), ROWS_D + ROWS_E + ROWS_F)
    worst = 0.0
    for t in range(T):
        d_h.upload(hs[t])
        ctx.run_moe(0, d_h.ptr, d_o.ptr)
        dec = d_o.download(np.float32)
        r = O.rel_to_scale(dec[rest].astype(np.float64), out[t][rest])
        worst = max(worst, r)
        assert r < TOL, (shared, t, r)
    ctx.check_error()
    print(f"batched wide passes ({shared} shared): {T} tokens, worst vs decode {worst:.2e}", flush=True)

