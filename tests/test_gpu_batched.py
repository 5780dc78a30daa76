"""The batched (multi-token) layer on the GPU (run with -m gpu): reference
run_moe_batched (src/glm_layer_runner.cuh:818-928), config 3.

Per token, the batched layer must agree with the numpy oracle and with the
single-token decode path (wl_run_moe, same routing arithmetic) within the
1e-5 rel_to_scale bar; passes of more than 32 tokens per expert are forced
with a strongly skewed router bias; repeated calls are bit-identical."""
import numpy as np
import pytest

from oracle import moe_oracle as O
from oracle import synth
from windlass_amd import hip as H_, synthdata
from windlass_amd.model import DeviceModel, make_io

pytestmark = pytest.mark.gpu
TOL = 1e-5
SMALL = dict(hidden=384, moe_inter=256, n_routed_experts=48, n_experts_per_tok=6, n_shared=1,
             routed_scaling=2.5, rms_eps=1e-5)
GLM = dict(hidden=6144, moe_inter=2048, n_routed_experts=256, n_experts_per_tok=8, n_shared=1,
           routed_scaling=2.5, rms_eps=1e-5)


def _tokens(H, T, seed):
    return np.stack([synth.hidden_state(H, seed, t) for t in range(T)]).astype(np.float32)


def _batched(dm, hs, resid=None):
    T, H = hs.shape
    dh = H_.DeviceBuffer.from_array(hs)
    dr = H_.DeviceBuffer.from_array(resid) if resid is not None else None
    do = H_.DeviceBuffer(4 * T * H)
    dm.ctx.run_moe_batched(0, T, dh.ptr, dr.ptr if dr else None, do.ptr)
    dm.ctx.check_error()
    return do.download(np.float32).reshape(T, H)


def _decode(dm, h):
    dh, dout = make_io(h.shape[0])
    dh.upload(h)
    dm.ctx.run_moe(0, dh.ptr, dout.ptr)
    dm.ctx.check_error()
    return dout.download(np.float32)


def _decode_routing(dm):
    """Logits, ids and weights of the last wl_run_moe (taps)."""
    tp = dm.ctx.taps()
    E, K = dm.cfg.n_routed_experts, dm.cfg.n_experts_per_tok
    return (H_.download_ptr(tp["logits"], np.float32, E), H_.download_ptr(tp["topk_idx"], np.int32, K),
            H_.download_ptr(tp["topk_w"], np.float32, K))


def _check_routing_bit_identical(dm, T, decode_routing):
    """The batched router (many tokens per work-group, wave sums taken
    together) performs the decode router's additions in the decode router's
    order: logits, ids (in order) and weights equal bit for bit."""
    lg, ids, w = dm.ctx.batched_routing(T)
    assert lg.shape[0] == T
    for t, (dl, di, dw) in enumerate(decode_routing):
        assert np.array_equal(lg[t].view(np.uint32), dl.view(np.uint32)), t
        assert np.array_equal(ids[t], di), t
        assert np.array_equal(w[t].view(np.uint32), dw.view(np.uint32)), t


@pytest.mark.parametrize("T", [1, 5, 33, 70])
def test_small_batched_vs_oracle_and_decode(gpu, T):
    c = SMALL
    H = c["hidden"]
    dm = DeviceModel(c, seed=12, n_layers=1)
    hs = _tokens(H, T, 300 + T)
    out = _batched(dm, hs)
    src = O.ExpertSource(H, c["moe_inter"], 12)
    worst = 0.0
    routing = []
    for t in range(T):
        dec = _decode(dm, hs[t])
        routing.append(_decode_routing(dm))
        r = O.rel_to_scale(dec, out[t])
        worst = max(worst, r)
        assert r < TOL, (t, r)
        if t < 3 or t == T - 1:
            ref = O.moe_layer(hs[t], dm.dense[0], src, 0, c)["out"]
            assert O.rel_to_scale(ref, out[t]) < TOL, t
    _check_routing_bit_identical(dm, T, routing)
    print(f"T={T}: worst batched-vs-decode rel_to_scale {worst:.2e}", flush=True)
    dm.close()


def test_skewed_routing_multi_pass_and_residual(gpu):
    """A bias that makes the same experts win for every token: those experts
    get all T tokens (several 32-token passes)."""
    c = SMALL
    H, E = c["hidden"], c["n_routed_experts"]
    off = np.zeros(E, np.float32)
    off[[3, 7, 11]] = 5.0
    dm = DeviceModel(c, seed=13, n_layers=1, bias_offset=off)
    T = 100
    hs = _tokens(H, T, 400)
    resid = _tokens(H, T, 401)
    out = _batched(dm, hs, resid)
    again = _batched(dm, hs, resid)
    assert np.array_equal(out, again)
    src = O.ExpertSource(H, c["moe_inter"], 13)
    for t in [0, 31, 32, 63, 64, 99]:
        ref = O.moe_layer(hs[t], dm.dense[0], src, 0, c)
        assert {3, 7, 11} <= set(int(i) for i in ref["topk_idx"])
        assert O.rel_to_scale(ref["out"], out[t] - resid[t]) < TOL, t
    dm.close()


def test_glm_batched_64_vs_decode(gpu):
    c = GLM
    H = c["hidden"]
    zipf = synthdata.zipf_bias_offset(c["n_routed_experts"], 14, amplitude=0.25)
    dm = DeviceModel(c, seed=14, n_layers=1, bias_offset=zipf)
    T = 64
    hs = _tokens(H, T, 500)
    out = _batched(dm, hs)
    worst = 0.0
    routing = []
    for t in range(T):
        r = O.rel_to_scale(_decode(dm, hs[t]), out[t])
        routing.append(_decode_routing(dm))
        worst = max(worst, r)
        assert r < TOL, (t, r)
    _check_routing_bit_identical(dm, T, routing)
    src = O.ExpertSource(H, c["moe_inter"], 14)
    ref = O.moe_layer(hs[5], dm.dense[0], src, 0, c)["out"]
    assert O.rel_to_scale(ref, out[5]) < TOL
    print(f"GLM T=64: worst batched-vs-decode rel_to_scale {worst:.2e}", flush=True)
    dm.close()


def _oracle_tokens(ids, T, kmt=32, want=10):
    """Tokens to check against the oracle: the first and the last, and tokens
    of the two experts with the most tokens (more than kmt of them, i.e. run
    in several passes): the first of each pass boundary and the last."""
    lists = {}
    for t in range(T):
        for e in ids[t]:
            lists.setdefault(int(e), []).append(t)
    hot = sorted(lists, key=lambda e: -len(lists[e]))[:2]
    pick = [0, T - 1]
    multi = []
    for e in hot:
        ts = lists[e]
        if len(ts) > kmt:
            multi.append(e)
            pick += [ts[kmt - 1], ts[kmt], ts[-1]]
    step = max(1, T // want)
    for t in range(step // 2, T, step):
        if len(set(pick)) >= want:
            break
        pick.append(t)
    return sorted(set(pick)), multi, {e: len(lists[e]) for e in hot}


@pytest.mark.parametrize("T", [256, 1024])
def test_glm_batched_zipf_vs_decode_and_oracle(gpu, T):
    """Config 3 at the GLM shape with the benchmark's Zipf(1.1) router bias:
    every token's routing equals the decode path's bit for bit and its output
    is within 1e-5 of the decode path's; at least 8 tokens (the first, the
    last, and tokens on both sides of a 32-token pass boundary of the busiest
    experts) are within 1e-5 of the oracle."""
    c = GLM
    H = c["hidden"]
    zipf = synthdata.zipf_bias_offset(c["n_routed_experts"], 15, amplitude=0.25)
    dm = DeviceModel(c, seed=15, n_layers=1, bias_offset=zipf)
    hs = _tokens(H, T, 600 + T)
    out = _batched(dm, hs)
    lg, ids, w = dm.ctx.batched_routing(T)
    counts = dm.ctx.batched_counts()
    assert int(counts.sum()) == T * c["n_experts_per_tok"]
    dh, dout = make_io(H)
    worst = 0.0
    tp = dm.ctx.taps()
    E, K = c["n_routed_experts"], c["n_experts_per_tok"]
    for t in range(T):
        dh.upload(hs[t])
        dm.ctx.run_moe(0, dh.ptr, dout.ptr)
        dm.ctx.check_error()
        dec = dout.download(np.float32)
        assert np.array_equal(lg[t].view(np.uint32), H_.download_ptr(tp["logits"], np.float32, E).view(np.uint32)), t
        assert np.array_equal(ids[t], H_.download_ptr(tp["topk_idx"], np.int32, K)), t
        assert np.array_equal(w[t].view(np.uint32), H_.download_ptr(tp["topk_w"], np.float32, K).view(np.uint32)), t
        r = O.rel_to_scale(dec, out[t])
        worst = max(worst, r)
        assert r < TOL, (t, r)
    pick, multi, hot = _oracle_tokens(ids, T)
    assert len(pick) >= 8
    assert multi, f"no expert ran more than one 32-token pass at T={T}: {hot}"
    src = O.ExpertSource(H, c["moe_inter"], 15, cache=48)
    worst_ref = 0.0
    for t in pick:
        ref = O.moe_layer(hs[t], dm.dense[0], src, 0, c)
        assert np.array_equal(np.sort(ref["topk_idx"]), np.sort(ids[t])), t
        r = O.rel_to_scale(ref["out"], out[t])
        worst_ref = max(worst_ref, r)
        assert r < TOL, (t, r)
    print(f"GLM T={T}: experts used {int((counts > 0).sum())}, busiest {hot}, "
          f"worst vs decode {worst:.2e}, worst vs oracle {worst_ref:.2e} over tokens {pick}", flush=True)
    dm.close()


def test_misaligned_or_aliasing_buffers_rejected(gpu):
    """The combine reads and writes rows 16 bytes at a time: buffers that are
    not 16-byte aligned are an argument error (nothing is launched), and so
    is an output that partly overlaps an input. Exact aliasing (the
    reference's in-place b.hidden update) runs and gives the out-of-place
    bits."""
    from windlass_amd.moe import WindlassError
    c = SMALL
    H = c["hidden"]
    dm = DeviceModel(c, seed=12, n_layers=1)
    T = 3
    dh = H_.DeviceBuffer(4 * T * H + 64)
    do = H_.DeviceBuffer(4 * T * H + 64)
    for args in [(dh.ptr, None, do.ptr + 4), (dh.ptr + 8, None, do.ptr), (dh.ptr, dh.ptr + 4, do.ptr),
                 (dh.ptr, None, dh.ptr + 4 * H)]:
        with pytest.raises(WindlassError) as ei:
            dm.ctx.run_moe_batched(0, T, *args)
        assert ei.value.status == 1, args  # WL_ERR_INVALID
    hs = _tokens(H, T, 450)
    dh.upload(hs)
    dm.ctx.run_moe_batched(0, T, dh.ptr, dh.ptr, do.ptr)  # aligned, out of place: runs
    dm.ctx.check_error()
    ref = do.download(np.float32, T * H)
    dm.ctx.run_moe_batched(0, T, dh.ptr, dh.ptr, dh.ptr)  # in place: hidden += moe(hidden)
    dm.ctx.check_error()
    assert np.array_equal(dh.download(np.float32, T * H).view(np.uint32), ref.view(np.uint32))
    dm.close()


def test_calls_longer_than_a_chunk(gpu):
    """A call of more than 4096 tokens runs in chunks of 4096 on the same
    scratch: 4,141 tokens with a residual give the same rows, bit for bit, as
    two calls over [0, 4096) and [4096, 4141), and agree within the bar with
    a call split elsewhere (other passes per expert), with the decode path
    around the boundary and with the oracle at both ends."""
    c = SMALL
    H = c["hidden"]
    T = 4096 + 45
    dm = DeviceModel(c, seed=14, n_layers=1)
    hs = _tokens(H, T, 1400)
    resid = _tokens(H, T, 1401)
    whole = _batched(dm, hs, resid)
    first = _batched(dm, hs[:4096], resid[:4096])
    rest = _batched(dm, hs[4096:], resid[4096:])
    assert np.array_equal(whole[:4096], first)
    assert np.array_equal(whole[4096:], rest)
    other = np.concatenate([_batched(dm, hs[:2000], resid[:2000]), _batched(dm, hs[2000:], resid[2000:])])
    worst = max(O.rel_to_scale(whole[t] - resid[t], other[t] - resid[t]) for t in range(T))
    assert worst < TOL, worst
    src = O.ExpertSource(H, c["moe_inter"], 14)
    for t in (0, 4094, 4095, 4096, 4097, T - 1):
        moe_t = whole[t] - resid[t]
        assert O.rel_to_scale(_decode(dm, hs[t]), moe_t) < TOL, t
        if t in (0, T - 1):
            ref = O.moe_layer(hs[t], dm.dense[0], src, 0, c)["out"]
            assert O.rel_to_scale(ref, moe_t) < TOL, t
    print(f"T={T}: chunked call equals per-chunk calls; worst vs another split {worst:.2e}", flush=True)
    dm.close()


@pytest.mark.parametrize("T", [64, 256])
def test_small_expert_units_equal_grouped_passes(gpu, monkeypatch, T):
    """At the GLM shape experts of up to 8 tokens run their gate/up and down
    as streaming units instead of grouped passes (the kernels' small-expert
    instantiations). WL_BATCHED_SMALL=0 keeps every
    expert in the grouped passes; both give the same outputs bit for bit,
    with the bench's Zipf bias (T = 64: most experts hold 1-4 tokens; 256:
    most hold 5-16)."""
    c = GLM
    H = c["hidden"]
    zipf = synthdata.zipf_bias_offset(c["n_routed_experts"], 1, amplitude=0.25)
    dm = DeviceModel(c, seed=1, n_layers=1, bias_offset=zipf)
    hs = _tokens(H, T, 1600)
    monkeypatch.delenv("WL_BATCHED_SMALL", raising=False)
    units = _batched(dm, hs)
    counts = dm.ctx.batched_counts()
    monkeypatch.setenv("WL_BATCHED_SMALL", "0")
    grouped = _batched(dm, hs)
    small = int(((counts >= 1) & (counts <= 8)).sum())
    print(f"T={T}: {small} experts of 1-8 tokens", flush=True)
    assert small > 20
    assert np.array_equal(units.view(np.uint32), grouped.view(np.uint32))
    dm.close()
