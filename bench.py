#!/usr/bin/env python3
"""Benchmark of the MoE decode hot path on one MI355X.

Workload: one GLM-style MoE decode layer at bs=1 —
hidden 6144, router bf16 [256,6144] + f32 bias, sigmoid / top-8 / renorm /
x2.5, 8 of 256 MXFP4 experts (inter 2048), one bf16 shared expert. A step is
one layer for one token. Steps rotate over --layers distinct layer copies
(each with its own 256 experts, router and shared expert, all resident in HBM)
so that the 256 MB Infinity Cache cannot serve a layer's weights from a
previous step; every step also has its own hidden state, so routing differs.

Prints ONE JSON line. `value` is microseconds per layer (lower is better),
measured with HIP events on the launch stream over the timed steps; the
roofline block divides the layer's algorithmic bytes by that time.

--workload chain measures BASELINE.json configs[2] instead: 24 resident GLM
MoE layers (6144 expert blocks, 123 GB of HBM), h <- h + moe(h) layer by
layer; a step is one decode token through all 24 layers, starting from its own
seeded N(0,1) hidden state. `value` is then microseconds per layer within the
chain (step time / 24) and tokens_per_s is reported beside it.

--workload batched measures configs[3]: one GLM MoE layer applied to
--tokens T positions at once (wl_run_moe_batched), router bias with the Zipf
offset; `value` is microseconds per layer call (all T tokens), with
tokens_per_s and the achieved bytes of the experts actually used.

--workload attention measures the caller side of a decoder layer (the
run_layer row): MLA attention with the DSA indexer at the GLM shape (hidden
6144, 64 heads, q_lora 2048, kv_lora 512, index_topk 2048) after --context
cached positions, over 4 rotating layers (two owning the indexer, two
sharing it); a step is one token through the 4 layers, `value` is
microseconds per attention layer; the dense MLP (intermediate 12288) is
timed beside it.

--workload files measures the file tier and the loader (rows f1, f4) at the
GLM shape: --file-layers packed layer_N.bin files written from the
synthetic generator to local disk, read through a --file-slots HBM cache by
4 pread workers: through the page cache with speculation off and on, and
with O_DIRECT; the same tokens then run through config 4's pinned-host cache
at the same layers and capacity, speculation off and on. Then a one-layer
safetensors checkpoint is loaded into the slot table (wl_load_layer +
wl_load_experts) and packed back into a layer file (wl_st_pack_layer). The
line reports hit rate, µs per layer and GB/s copied of each pass; the files
are removed at the end.

--workload cache measures configs[4]: 75 MoE layers whose 19,200 experts sit
behind the HBM expert cache (3,094 slots, 62 GB) and are copied from pinned
host memory on a miss; router bias shaped by Zipf(1.1) popularity; a step is
one token through the 75 layers; --spec adds cross-layer speculative prefetch. The host backing store is --host-blocks pinned native blocks
(default 512, 10.3 GB): (layer, expert) reads block (layer*256 + expert) mod
512, because 385 GB of distinct blocks exceed the host memory of the box. The
key, the LRU and every copy are per (layer, expert) as in the reference; only
the bytes repeat. The line adds hit_rate and the host-link rate.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBPS = 8000.0
GLM = dict(hidden=6144, moe_inter=2048, n_routed_experts=256, n_experts_per_tok=8, n_shared=1,
           routed_scaling=2.5, rms_eps=1e-5)


def algorithmic_bytes(c, shared_mxfp4=False):
    """Bytes one decode layer must move at least once: K expert blocks, the
    shared expert (bf16, or one MXFP4 block of inter SI), the bf16 router,
    the f32 bias, the f32 input and output vectors."""
    H, I, E, K = c["hidden"], c["moe_inter"], c["n_routed_experts"], c["n_experts_per_tok"]
    SI = I * c["n_shared"]
    expert = 3 * I * H // 2 + 3 * I * H // 32
    shared = 3 * SI * H // 2 + 3 * SI * H // 32 if shared_mxfp4 else 3 * SI * H * 2
    return K * expert + shared + E * H * 2 + E * 4 + 2 * H * 4


def host_cores():
    """(physical cores, logical CPUs) this process may run on: the distinct
    (core, socket) pairs lscpu lists for the CPUs of the affinity set."""
    import subprocess
    cpus = os.sched_getaffinity(0)
    try:
        out = subprocess.run(["lscpu", "-p=CPU,CORE,SOCKET"], capture_output=True, text=True, check=True).stdout
        pairs = set()
        for ln in out.splitlines():
            if ln.startswith("#"):
                continue
            cpu, core, sock = ln.split(",")[:3]
            if int(cpu) in cpus:
                pairs.add((core, sock))
        phys = len(pairs) or len(cpus)
    except (OSError, ValueError, subprocess.CalledProcessError):
        phys = len(cpus)
    return phys, len(cpus)


def cpu_baseline_batched(c, seed, hb, bias_offset, threads, n_expert_sample=3, n_apply_sample=8,
                         n_route_sample=32, n_shared_sample=4):
    """The reference's batched layer on the CPU (tools/ref_glm_chain.py:789-868,
    passes 2-4: route every position, then EXPERT-major: each routed expert
    dequantised once and applied position by position with matvecs, then the
    per-position combine), timed on a bounded sample and extrapolated:
    routing per position (first n_route_sample positions), dequant per expert
    and per-position expert applications (the first n_expert_sample experts in
    sorted order, up to n_apply_sample applications each), shared expert per
    position (n_shared_sample positions). Returns (us per call, sample text)."""
    from threadpoolctl import threadpool_limits

    from oracle import moe_oracle as O
    from oracle import synth
    H, I, E, K = c["hidden"], c["moe_inter"], c["n_routed_experts"], c["n_experts_per_tok"]
    T = hb.shape[0]
    dense = synth.dense_layer(H, E, I * c["n_shared"], seed, 0)
    bias = (dense["bias"] + bias_offset).astype(np.float32)
    rw = synth.bf16_to_f32(dense["router_w"]).reshape(E, H)
    SG, SU, SD = O.shared_matrices(dense, H, I * c["n_shared"])
    with threadpool_limits(limits=threads):
        prep = []
        t0 = time.perf_counter()
        for t in range(T):
            xn = O.rms_norm(hb[t], None, c["rms_eps"])
            _, idx, wt, _ = O.route(xn, rw, bias, K, c["routed_scaling"], True)
            prep.append((xn, idx, wt))
            if t + 1 == n_route_sample:
                t_route = (time.perf_counter() - t0) / n_route_sample
        if T < n_route_sample:
            t_route = (time.perf_counter() - t0) / T
        routed = {}
        for t, (_, idx, _) in enumerate(prep):
            for k, e in enumerate(idx):
                routed.setdefault(int(e), []).append((t, k))
        t_deq, t_app = [], []
        for e in sorted(routed)[:n_expert_sample]:
            gw, gs, uw, us, dw, ds = synth.expert_block(H, I, seed, 0, e)
            t0 = time.perf_counter()
            G, U, D = O.dequant(gw, gs), O.dequant(uw, us), O.dequant(dw, ds)
            t_deq.append(time.perf_counter() - t0)
            for t, k in routed[e][:n_apply_sample]:
                t0 = time.perf_counter()
                O.expert_slot(prep[t][0], G, U, D)
                t_app.append(time.perf_counter() - t0)
        t_sh = []
        for t in range(min(T, n_shared_sample)):
            t0 = time.perf_counter()
            O.silu(prep[t][0] @ SG.T) * (prep[t][0] @ SU.T) @ SD.T
            t_sh.append(time.perf_counter() - t0)
    uniq = len(routed)
    total = (t_route * T + float(np.mean(t_deq)) * uniq + float(np.median(t_app)) * T * K
             + float(np.median(t_sh)) * T)
    text = (f"numpy oracle in the reference's batched order (route every position; each of the {uniq} experts "
            f"dequantised once, then {T * K} per-position expert matvec applications; shared expert per position); "
            f"timed on routing of {min(T, n_route_sample)} positions, dequant of {len(t_deq)} experts, "
            f"{len(t_app)} expert applications and {len(t_sh)} shared applications, extrapolated to T={T}")
    return total * 1e6, text


def cpu_baseline(c, seed, n_layers_sample, threads):
    """The numpy oracle (the reference's algorithm: dequantise to fp32, then
    BLAS matvecs; tools/ref_glm_chain.py:646-711) on this host, over a small
    sample of layers. Returns microseconds per layer (median)."""
    from threadpoolctl import threadpool_limits

    from oracle import moe_oracle as O
    from oracle import synth
    H, I, E = c["hidden"], c["moe_inter"], c["n_routed_experts"]
    dense = synth.dense_layer(H, E, I * c["n_shared"], seed, 0)
    sh = O.shared_matrices(dense, H, I * c["n_shared"])
    blocks = {}
    times = []
    with threadpool_limits(limits=threads):
        for step in range(n_layers_sample + 1):
            h = synth.hidden_state(H, 1000 + step)
            # packed expert bytes are read from memory (not timed: the reference
            # reads them from its packed files); dequant + matvecs are timed
            xn = O.rms_norm(h, None, c["rms_eps"])
            rw = synth.bf16_to_f32(dense["router_w"]).reshape(E, H)
            _, idx, _, _ = O.route(xn, rw, dense["bias"], c["n_experts_per_tok"], 2.5, True)
            for e in idx:
                if int(e) not in blocks:
                    blocks[int(e)] = synth.expert_block(H, I, seed, 0, int(e))

            class Src:
                def get(self, layer, e):
                    gw, gs, uw, us, dw, ds = blocks[e]
                    return O.dequant(gw, gs), O.dequant(uw, us), O.dequant(dw, ds)

            t0 = time.perf_counter()
            O.moe_layer(h, dense, Src(), 0, c, shared_f32=sh)
            dt = time.perf_counter() - t0
            if step > 0:  # first run is the warm-up
                times.append(dt)
    return float(np.median(times)) * 1e6, len(times)


GLM_ATTN = dict(hidden=6144, n_heads=64, q_lora_rank=2048, kv_lora_rank=512, qk_nope=192, qk_rope=64, v_head=256,
                index_n_heads=32, index_head_dim=128, index_topk=2048, dense_inter=12288, rms_eps=1e-5,
                rope_theta=1e6)


def attention_bytes(a, T, owner):
    """Bytes one decode attention layer must move at T cached keys: its bf16
    projections (the indexer's on owning layers, weights_proj f32), the KV
    cache rows (kv_c | k_rot f32) and, on owning layers, the indexer keys."""
    H, HN, Q, L = a["hidden"], a["n_heads"], a["q_lora_rank"], a["kv_lora_rank"]
    NP, RP, VD, IH, ID = a["qk_nope"], a["qk_rope"], a["v_head"], a["index_n_heads"], a["index_head_dim"]
    w = 2 * (Q * H + HN * (NP + RP) * Q + (L + RP) * H + HN * (NP + VD) * L + H * HN * VD) + 2 * H
    kv = 4 * T * (L + RP)
    if owner:
        w += 2 * (IH * ID * Q + ID * H) + 4 * IH * H
        kv += 4 * T * ID
    return w + kv + 2 * 4 * H


def cpu_baseline_attention(a, T, threads, n_sample=3):
    """The numpy oracle's step (oracle/attention.py attn_block: projections,
    indexer, attention over T cached keys, o_proj) on one owning layer with
    T - 1 rows of random cache; median of n_sample positions after one
    warm-up."""
    from threadpoolctl import threadpool_limits

    from oracle import attention as A
    from windlass_amd import synthdata
    W = synthdata.as_f32(synthdata.attention_layer(a, 1, 0, owner=True))
    rng = np.random.default_rng(0)
    HN, DH, VD, ID = a["n_heads"], a["qk_nope"] + a["qk_rope"], a["v_head"], a["index_head_dim"]
    cache = A.LayerCache()
    cache.k = list(rng.standard_normal((T - 1, HN, DH), dtype=np.float32))
    cache.v = list(rng.standard_normal((T - 1, HN, VD), dtype=np.float32))
    cache.ik = list(rng.standard_normal((T - 1, ID), dtype=np.float32))
    cos, sin = A.rope_tables(T + n_sample + 1, a["qk_rope"], a["rope_theta"])
    times = []
    with threadpool_limits(limits=threads):
        for i in range(n_sample + 1):
            h = synthdata.hidden_state(a["hidden"], 9000 + i)
            t0 = time.perf_counter()
            A.attn_block(h, W, a, T - 1, cos, sin, cache, True, A.IndexShare())
            if i > 0:
                times.append(time.perf_counter() - t0)
            for lst in (cache.k, cache.v, cache.ik):
                lst.pop()
    return float(np.median(times)) * 1e6, len(times)


def bench_attention(args):
    from windlass_amd import hip
    from windlass_amd.model import AttnModel
    a = dict(GLM_ATTN)
    H = a["hidden"]
    if "--steps" not in sys.argv:
        args.steps = 200
    if "--warmup" not in sys.argv:
        args.warmup = 10
    n_l = 4
    owners = [True, False, True, False]
    t_build = time.time()
    am = AttnModel(a, args.seed, n_l, owners=owners, dense=[0, 1], max_seq=args.context + args.warmup + args.steps + 1)
    n_h = 64
    d_hs = hip.DeviceBuffer.from_array(np.stack([synthdata_hidden(H, 5000 + i) for i in range(n_h)]))
    d_h = hip.DeviceBuffer(4 * H)
    stream = hip.Stream()
    # fill the KV caches: positions 0 .. context-1 through every layer
    for pos in range(args.context):
        hip.copy_d2d(d_h.ptr, d_hs.ptr + 4 * H * (pos % n_h), 4 * H, stream.handle)
        for l in range(n_l):
            am.attn.run_attention(l, pos, d_h.ptr, stream.handle)
    stream.synchronize()
    build_s = time.time() - t_build

    def token(pos):
        hip.copy_d2d(d_h.ptr, d_hs.ptr + 4 * H * (pos % n_h), 4 * H, stream.handle)
        for l in range(n_l):
            am.attn.run_attention(l, pos, d_h.ptr, stream.handle)

    pos = args.context
    for i in range(args.warmup):
        token(pos)
        pos += 1
    stream.synchronize()
    e0, e1 = hip.Event(), hip.Event()
    e0.record(stream)
    for i in range(args.steps):
        token(pos)
        pos += 1
    e1.record(stream)
    e1.synchronize()
    us_layer = e0.elapsed_ms(e1) * 1e3 / args.steps / n_l
    T = pos - args.steps // 2  # mean cached keys of the timed tokens
    nbytes = (attention_bytes(a, T, True) + attention_bytes(a, T, False)) / 2
    achieved = nbytes / (us_layer * 1e-6) / 1e9
    # dense MLP beside it (two rotating layers)
    for i in range(args.warmup):
        am.attn.run_dense_mlp(i % 2, d_h.ptr, stream.handle)
    e0.record(stream)
    for i in range(args.steps):
        am.attn.run_dense_mlp(i % 2, d_h.ptr, stream.handle)
    e1.record(stream)
    e1.synchronize()
    us_mlp = e0.elapsed_ms(e1) * 1e3 / args.steps
    mlp_bytes = 3 * a["dense_inter"] * H * 2 + H * 2 + 2 * 4 * H
    cpu = None
    if args.cpu_sample > 0:
        phys, logical = host_cores()
        ncores = min(phys, 16)
        us_all, n_all = cpu_baseline_attention(a, T, ncores)
        cpu = {"value": round(us_all, 1), "unit": "us/layer", "cores": ncores, "kind": "port",
               "sample": f"numpy oracle attn_block (projections, indexer, attention over {T} keys, o_proj) on one "
                         f"indexer-owning layer, median of {n_all} positions after one warm-up",
               "host_physical_cores": phys, "host_logical_cpus": logical, "gpu_speedup": round(us_all / us_layer, 1)}
    line = {
        "metric": "us_per_attention_layer",
        "value": round(us_layer, 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_layer * n_l / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 weights, f32 activations, KV cache and accumulation",
        "data": "synthetic",
        "config": {"workload": f"run_layer attention side: MLA + DSA indexer, decode at {args.context}+ cached "
                               f"positions, 4 rotating layers (2 indexer-owning, 2 sharing)", **a},
        "achieved_GBps": round(achieved, 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBPS, 4), "traffic": None,
                     "algorithmic_bytes": int(nbytes), "kernel": "whole attention layer (gemv_kernel dominates)"},
        "dense_mlp": {"us_per_layer": round(us_mlp, 3), "algorithmic_bytes": mlp_bytes,
                      "achieved_GBps": round(mlp_bytes / (us_mlp * 1e-6) / 1e9, 1),
                      "frac": round(mlp_bytes / (us_mlp * 1e-6) / 1e9 / PEAK_HBM_GBPS, 4)},
        "cpu_baseline": cpu,
        "build_s": round(build_s, 1),
    }
    am.close()
    print(json.dumps(line), flush=True)


def bench_files(args):
    import shutil
    import tempfile

    from windlass_amd import checkpoint, hip, moe, synthdata
    from windlass_amd.model import CachedModel, FileModel
    c = dict(GLM)
    H, I, E = c["hidden"], c["moe_inter"], c["n_routed_experts"]
    L = args.file_layers
    work = tempfile.mkdtemp(prefix="wl_files_", dir=args.file_dir)
    out = {}
    try:
        cfg = moe.make_config(hidden=H, moe_inter=I, n_routed_experts=E, n_experts_per_tok=c["n_experts_per_tok"],
                              n_shared=1, n_layers=L)
        blk = moe.expert_layout(cfg).total
        d_ref, h_ref = hip.DeviceBuffer(blk), hip.HostBuffer(blk)

        def expert_bytes(l, e):
            moe.synth_expert(cfg, args.seed, l, e, d_ref.ptr)
            hip.copy_d2h_ptr(h_ref.ptr, d_ref.ptr, blk)
            return h_ref.view(np.uint8, blk)

        t0 = time.time()
        for l in range(L):
            with open(os.path.join(work, f"layer_{l}.bin"), "wb") as f:
                for e in range(E):
                    f.write(expert_bytes(l, e).tobytes())
        out["write_s"] = round(time.time() - t0, 1)
        zipf = synthdata.zipf_bias_offset(E, args.seed, amplitude=args.zipf_amp)
        n_h = 64
        d_hs = hip.DeviceBuffer.from_array(np.stack([synthdata.hidden_state(H, 5000 + i) for i in range(n_h)]))
        d_h, d_tmp = hip.DeviceBuffer(4 * H), hip.DeviceBuffer(4 * H)
        stream = hip.Stream()
        # the same tokens through every pass, so the routed keys (and the
        # LRU's hits and misses without speculation) are the same in each;
        # "pinned_host" is config 4's path (native blocks in pinned host
        # memory, aliased over 512 blocks) at the same layers and capacity
        passes = (("page_cache", "files", False, False, 16, 4), ("page_cache_spec", "files", False, True, 16, 4),
                  ("direct", "files", True, False, 4, 2), ("pinned_host", "host", False, False, 16, 4),
                  ("pinned_host_spec", "host", False, True, 16, 4))
        for name, kind, direct, spec, steps, warm in passes:
            print(f"bench files: {name}, {L} layers, {args.file_slots} slots, {steps} tokens", file=sys.stderr,
                  flush=True)
            if kind == "files":
                fm = FileModel(c, args.seed, L, capacity=args.file_slots, directory=work, io_threads=4,
                               shared_alias=True, bias_offset=zipf, direct=direct)
            else:
                fm = CachedModel(c, args.seed, L, capacity=args.file_slots, n_host=min(L * E, 512),
                                 shared_alias=True, bias_offset=zipf)
            fm.ctx.set_taps(False)
            fm.ctx.cache_set_speculation(spec)

            def token(i):
                hip.copy_d2d(d_h.ptr, d_hs.ptr + 4 * H * (i % n_h), 4 * H, stream.handle)
                fm.ctx.run_chain(0, L, d_h.ptr, d_tmp.ptr, stream.handle)

            for i in range(warm):
                token(i)
            stream.synchronize()
            fm.ctx.cache_reset_stats()
            e0, e1 = hip.Event(), hip.Event()
            e0.record(stream)
            for i in range(steps):
                token(warm + i)
            e1.record(stream)
            e1.synchronize()
            ms = e0.elapsed_ms(e1)
            fm.ctx.check_error(stream.handle)
            st = fm.ctx.cache_stats()
            req = st["hits"] + st["misses"]
            copied = st["bytes_h2d"]
            out[name] = {
                "us_per_layer": round(ms * 1e3 / steps / L, 1), "tokens": steps,
                "tokens_per_s": round(steps / (ms * 1e-3), 2),
                "hit_rate": round(st["hits"] / max(1, req), 4), "misses": st["misses"],
                "spec_copies": st["spec_copies"], "spec_hits": st["spec_hits"],
                "GBps_copied": round(copied / (ms * 1e-3) / 1e9, 2)}
            fm.close()
        # loader: a one-layer checkpoint (dense fields + 256 experts) -> slot table, and -> packed file
        d = synthdata.dense_layer(H, E, I, args.seed, 0)
        P = "model.layers.0."
        lay = moe.expert_layout(cfg)
        parts = [(lay.gw_off, lay.gw_len, (I, H // 2)), (lay.gs_off, lay.gs_len, (I, H // 32)),
                 (lay.uw_off, lay.uw_len, (I, H // 2)), (lay.us_off, lay.us_len, (I, H // 32)),
                 (lay.dw_off, lay.dw_len, (H, I // 2)), (lay.ds_off, lay.ds_len, (H, I // 32))]
        names = ["gate_proj.weight", "gate_proj.weight_scale", "up_proj.weight", "up_proj.weight_scale",
                 "down_proj.weight", "down_proj.weight_scale"]
        ts = [(P + "post_attention_layernorm.weight", "BF16", (H,), np.full(H, 0x3F80, np.uint16)),
              (P + "mlp.gate.weight", "BF16", (E, H), d["router_w"]),
              (P + "mlp.gate.e_score_correction_bias", "F32", (E,), d["bias"]),
              (P + "mlp.shared_experts.gate_proj.weight", "BF16", (I, H), d["sh_gate"]),
              (P + "mlp.shared_experts.up_proj.weight", "BF16", (I, H), d["sh_up"]),
              (P + "mlp.shared_experts.down_proj.weight", "BF16", (H, I), d["sh_down"])]
        cur = {}

        def part_of(e, j):
            def f():
                if cur.get("e") != e:
                    cur["e"], cur["b"] = e, expert_bytes(0, e).copy()
                off, n, _ = parts[j]
                return cur["b"][off:off + n]
            return f

        for e in range(E):
            for j in range(6):
                ts.append((f"{P}mlp.experts.{e}.{names[j]}", "U8", parts[j][2], (part_of(e, j), parts[j][1])))
        ck = os.path.join(work, "ckpt")
        checkpoint.write_checkpoint(ck, ts, n_shards=1)
        c1 = moe.make_config(hidden=H, moe_inter=I, n_routed_experts=E, n_experts_per_tok=c["n_experts_per_tok"],
                             n_shared=1, n_layers=1)
        ctx = moe.Context(c1)
        ctx.slot_pool_create(E)
        t0 = time.time()
        st = moe.SafeTensors(ck)
        t_open = time.time() - t0
        t0 = time.time()
        ctx.load_layer(st, 0, 0)
        t_layer = time.time() - t0
        t0 = time.time()
        ctx.load_experts(st, 0, 0, n=E, first_slot=0)
        t_exp = time.time() - t0
        t0 = time.time()
        st.pack_layer(c1, 0, os.path.join(work, "packed_0.bin"))
        t_pack = time.time() - t0
        out["loader"] = {"open_ms": round(t_open * 1e3, 1), "load_layer_ms": round(t_layer * 1e3, 1),
                         "load_experts_s": round(t_exp, 3), "load_experts_GBps": round(E * blk / t_exp / 1e9, 2),
                         "pack_layer_s": round(t_pack, 3), "pack_layer_GBps": round(E * blk / t_pack / 1e9, 2),
                         "note": "checkpoint just written: read through the page cache"}
        ctx.close()
        st.close()
    finally:
        shutil.rmtree(work, ignore_errors=True)
    line = {"metric": "file_tier_GBps", "value": out["page_cache"]["GBps_copied"], "unit": "GB/s", "n_gpus": 1,
            "higher_is_better": True, "data": "synthetic", "dtype": "mxfp4 expert records",
            "config": {"workload": f"file tier: {L} GLM layer files ({L * E} records of {blk} B), "
                                   f"{args.file_slots}-slot HBM cache, 4 pread workers, bs=1 tokens",
                       "zipf_amplitude": args.zipf_amp},
            **out}
    print(json.dumps(line), flush=True)


def bench_expert(args):
    """Config 0: one MXFP4 expert SwiGLU FFN at bs=1 (wl_expert_ffn: gate/up +
    SwiGLU, then down), over 64 reference-layout blocks (8 seeds x 8 experts,
    1.28 GB) rotated so that no step finds its block in the 256 MB Infinity
    Cache, each step with its own bf16 N(0,1) input."""
    import ctypes

    from windlass_amd import hip, moe, synthdata
    c = dict(GLM)
    H, I = c["hidden"], c["moe_inter"]
    cfg = moe.make_config(hidden=H, moe_inter=I, n_routed_experts=c["n_routed_experts"],
                          n_experts_per_tok=c["n_experts_per_tok"], n_shared=1, n_layers=1)
    ctx = moe.Context(cfg)
    lay = moe.expert_layout(cfg)
    seeds, per_seed = 8, 8
    nblk = seeds * per_seed
    pool = hip.DeviceBuffer(nblk * lay.total)
    for s in range(seeds):
        for e in range(per_seed):
            moe.synth_expert(cfg, s, 0, e, pool.ptr + (s * per_seed + e) * lay.total)
    hip.synchronize()
    n_x = 16
    xs = np.stack([synthdata.hidden_state(H, 8000 + i) for i in range(n_x)])
    d_x = hip.DeviceBuffer.from_array(xs)
    d_y = hip.DeviceBuffer(4 * H * n_x)
    stream = hip.Stream()
    lib = moe.load()

    def step(i):
        b = i % nblk
        rc = lib.wl_expert_ffn(ctx.h, pool.ptr + b * lay.total, d_x.ptr + 4 * H * (i % n_x),
                               d_y.ptr + 4 * H * (i % n_x), None, stream.handle)
        if rc != moe.WL_OK:
            raise moe.WindlassError(rc, "wl_expert_ffn")

    for i in range(args.warmup):
        step(i)
    ctx.check_error(stream.handle)
    hip.synchronize()
    e0, e1 = hip.Event(), hip.Event()
    e0.record(stream)
    for i in range(args.steps):
        step(args.warmup + i)
    e1.record(stream)
    e1.synchronize()
    us = e0.elapsed_ms(e1) * 1e3 / args.steps
    ctx.check_error(stream.handle)
    nbytes = lay.total + 2 * 4 * H  # the block, the f32 input and output
    achieved = nbytes / (us * 1e-6) / 1e9

    cpu = None
    if args.cpu_sample > 0:
        from oracle import moe_oracle as O
        phys, logical = host_cores()
        ncores = min(phys, 16)

        from threadpoolctl import threadpool_limits

        from oracle import synth
        # packed expert bytes are generated beforehand (not timed: the
        # reference reads them from its packed files); dequant + matvecs are
        blocks = [synth.expert_block(H, I, k % seeds, 0, k % per_seed) for k in range(min(args.cpu_sample + 1, 4))]

        def cpu_leg(threads):
            times = []
            with threadpool_limits(limits=threads):
                for k in range(args.cpu_sample + 1):
                    gw, gs, uw, us_, dw, ds = blocks[k % len(blocks)]
                    t0 = time.perf_counter()
                    O.expert_slot(xs[k % n_x], O.dequant(gw, gs), O.dequant(uw, us_), O.dequant(dw, ds))
                    times.append(time.perf_counter() - t0)
            return float(np.median(times[1:])) * 1e6

        us_all = cpu_leg(ncores)
        us_one = cpu_leg(1)
        cpu = {"value": round(us_all, 1), "unit": "us/expert", "cores": ncores, "kind": "port",
               "sample": f"numpy oracle (dequant to f32 + OpenBLAS matvecs) on {args.cpu_sample} expert FFNs after one "
                         f"warm-up, median; expert bytes pre-generated",
               "host_physical_cores": phys, "host_logical_cpus": logical, "value_1thread": round(us_one, 1),
               "gpu_speedup": round(us_all / us, 1)}
    line = {
        "metric": "us_per_mxfp4_expert_ffn", "value": round(us, 3), "unit": "us/expert", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(us / 1e3, 6), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "mxfp4 weights widened exactly to f32, f32 activations and accumulation",
        "data": "synthetic",
        "config": {"workload": "config0: one MXFP4 expert SwiGLU FFN, bs=1 (wl_expert_ffn)", "hidden": H,
                   "moe_inter": I, "rotating_blocks": nblk, "seeds": seeds, "global_batch": 1},
        "achieved_GBps": round(achieved, 1), "pct_of_hbm_peak": round(100 * achieved / PEAK_HBM_GBPS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBPS, 4), "traffic": None, "algorithmic_bytes": nbytes,
                     "kernel": "ffn1_kernel (one persistent launch)"},
        "cpu_baseline": cpu,
    }
    ctx.close()
    print(json.dumps(line), flush=True)


def bench_shim(args):
    """The drop-in shim (include/windlass_glm.hpp) driven by the reference's
    own call sites: tests/shim/_build/reference_caller runs decode steps of
    one dense layer and --shim-layers MoE layers at the GLM shape (shared
    expert in the checkpoint's MXFP4 format, as the reference's LayerWeights
    hold it), once with the experts made resident on first use and once with
    every expert fetched through the caller's ExpertSource (reference-layout
    blocks, converted per call). Runs as a child process; this process does
    not touch the GPU."""
    import contextlib
    import subprocess
    import tempfile

    from windlass_amd import synthdata
    binary = os.path.join(ROOT, "tests", "shim", "_build", "reference_caller")
    if not os.path.exists(binary):
        print(f"bench.py: {binary} is missing (run __graft_entry__.build())", file=sys.stderr)
        sys.exit(1)
    c = dict(GLM)
    H, I, E, K = c["hidden"], c["moe_inter"], c["n_routed_experts"], c["n_experts_per_tok"]
    DI, NL, T, seed = 12288, 1 + args.shim_layers, 16, args.seed
    res = {}
    keep = args.shim_dir
    if keep:
        os.makedirs(keep, exist_ok=True)
    with (contextlib.nullcontext(keep) if keep else tempfile.TemporaryDirectory()) as d:
        with open(os.path.join(d, "cfg.txt"), "w") as f:
            f.write(f"{NL} 1 {H} {I} {E} {K} 1 {DI} {T} {seed} {c['rms_eps']} {c['routed_scaling']}\n")
        w = synthdata.dense_mlp(H, DI, seed, 0)
        for k, name in (("post_ln", "ln"), ("gate", "gate"), ("up", "up"), ("down", "down")):
            w[k].tofile(os.path.join(d, f"l0_{name}.bin"))
        del w
        for l in range(1, NL):
            r = synthdata.router_only(H, E, seed, l)
            r["router_w"].tofile(os.path.join(d, f"l{l}_router.bin"))
            r["bias"].tofile(os.path.join(d, f"l{l}_bias.bin"))
            synthdata._norm_w(seed, l, synthdata.TAG_LN, H).tofile(os.path.join(d, f"l{l}_ln.bin"))
        np.stack([synthdata.hidden_state(H, 9000 + t) for t in range(T)]).astype(np.float32).tofile(
            os.path.join(d, "h0.bin"))
        for mode in ("resident", "source"):
            print(f"bench shim: {mode}, {NL} layers, {args.steps} steps", file=sys.stderr, flush=True)
            r = subprocess.run([binary, d, mode, str(args.steps)], capture_output=True, text=True, timeout=900)
            if r.returncode != 0:
                print(r.stdout + r.stderr, file=sys.stderr)
                sys.exit(r.returncode)
            res[mode] = json.loads(r.stdout.strip().splitlines()[-1])
    us = res["resident"]["us_per_moe_layer"]
    nbytes = algorithmic_bytes(c, shared_mxfp4=True)
    achieved = nbytes / (us * 1e-6) / 1e9
    dense_bytes = 3 * DI * H * 2 + H * 2 + 2 * H * 4
    line = {
        "metric": "us_per_moe_decode_layer", "value": round(us, 3), "unit": "us/layer", "n_gpus": 1,
        "steps": args.steps, "warmup": 2, "ms_per_step": round(res["resident"]["wall_us_per_step"] / 1e3, 6),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "mxfp4/bf16 weights, f32 activations and accumulation; the decode kernel's cross-work-group partial "
                 "sums are exchanged as f32 rounded to 21 stored mantissa bits", "data": "synthetic",
        "config": {"workload": f"shim: the reference's run_layer/run_chain call sites through include/windlass_glm.hpp, "
                               f"1 dense + {args.shim_layers} MoE GLM layers per decode step, MXFP4 shared expert",
                   "hidden": H, "moe_inter": I, "n_routed_experts": E, "n_experts_per_tok": K, "dense_inter": DI,
                   "global_batch": 1},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBPS, 4), "traffic": None, "algorithmic_bytes": nbytes,
                     "kernel": "moe_decode_kernel (resident MoE layer through the shim)"},
        "shim": {"resident_us_per_moe_layer": res["resident"]["us_per_moe_layer"],
                 "source_us_per_moe_layer": res["source"]["us_per_moe_layer"],
                 "dense_us_per_layer": res["resident"]["us_per_dense_layer"],
                 "dense_GBps": round(dense_bytes / (res["resident"]["us_per_dense_layer"] * 1e-6) / 1e9, 1),
                 "source_note": "every MoE call routes on the device, reads the ids back (one host round trip), "
                                "fetches 8 reference-layout blocks from the caller's ExpertSource and converts "
                                "each into the native layout before the decode kernel"},
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)


def synthdata_hidden(H, seed):
    from windlass_amd import synthdata
    return synthdata.hidden_state(H, seed)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--layers", type=int, default=8, help="distinct resident layer copies to rotate over")
    ap.add_argument("--sched", choices=["fused", "phased"], default="fused")
    ap.add_argument("--workload", choices=["layer", "chain", "batched", "cache", "attention", "files", "expert", "shim"],
                    default="layer",
                    help="layer: config 1 (default); chain: config 2, 24 layers per step; "
                         "batched: config 3, --tokens positions per step; cache: config 4, 75 cache-backed layers per step")
    ap.add_argument("--tokens", type=int, default=256, help="batched workload: positions per layer call")
    ap.add_argument("--noalloc", action="store_true",
                    help="batched workload: through wl_run_moe_batched_noalloc (static scratch, token chunks of its "
                         "capacity) instead of wl_run_moe_batched")
    ap.add_argument("--chain-layers", type=int, default=24)
    ap.add_argument("--cache-layers", type=int, default=75)
    ap.add_argument("--cache-slots", type=int, default=3094)
    ap.add_argument("--host-blocks", type=int, default=512)
    ap.add_argument("--spec", action="store_true",
                    help="cache workload: cross-layer speculative prefetch (layer l+1's router on layer l's input)")
    ap.add_argument("--policies", default="lru",
                    help="cache workload: comma-separated replacement/admission policies (lru, lfu, slru, 2q, "
                         "tinylfu), each measured on a flushed cache in turn; the first is the line's value")
    ap.add_argument("--pin-top", type=int, default=0,
                    help="cache workload: pin the N keys requested most often by a profile pass over the warm-up "
                         "tokens (popularity pinning)")
    ap.add_argument("--zipf-amp", type=float, default=0.25,
                    help="cache workload: bias offset of the most popular expert (rank r gets amp * r^-1.1)")
    ap.add_argument("--file-layers", type=int, default=2, help="files workload: packed layer files")
    ap.add_argument("--file-slots", type=int, default=64, help="files workload: HBM cache slots")
    ap.add_argument("--file-dir", default=None, help="files workload: directory for the files (default: a temp dir)")
    ap.add_argument("--context", type=int, default=4096,
                    help="attention workload: cached positions before the timed tokens")
    ap.add_argument("--shim-layers", type=int, default=4, help="shim workload: MoE layers after the dense one")
    ap.add_argument("--shim-dir", default=None,
                    help="shim workload: write the caller's inputs here and keep them (default: a temp dir), so that "
                         "tests/shim/_build/reference_caller DIR resident|source STEPS can be profiled on its own")
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--shared", choices=["bf16", "mxfp4"], default="bf16",
                    help="layer/chain workloads: the shared expert's format (bf16, the benchmark configuration; "
                         "mxfp4 is the checkpoint's own format)")
    ap.add_argument("--cpu-sample", type=int, default=6,
                    help="layers timed for the CPU baseline after one warm-up, median reported (0: skip)")
    ap.add_argument("--traffic-json", default=os.path.join(ROOT, "profiles", "decode_layer_traffic.json"))
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="after the timed steps, one device-to-device copy of this many MiB (the reference "
                         "transfer for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE counters)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}); "
              "the multi-GPU sharding of the MoE layer is not built.", file=sys.stderr)
        sys.exit(2)

    if args.workload == "shim":  # a child process drives the GPU
        if "--steps" not in sys.argv:
            args.steps = 40
        return bench_shim(args)

    from windlass_amd import hip, moe, synthdata
    from windlass_amd.model import CachedModel, DeviceModel

    if hip.device_count() < 1:
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.workload == "attention":
        return bench_attention(args)
    if args.workload == "files":
        return bench_files(args)
    if args.workload == "expert":
        return bench_expert(args)

    c = dict(GLM)
    H = c["hidden"]
    cache = args.workload == "cache"
    sh4 = args.shared == "mxfp4" and args.workload in ("layer", "chain")
    batched = args.workload == "batched"
    chain = args.workload == "chain" or cache
    if chain:
        args.layers = args.cache_layers if cache else args.chain_layers
        if "--steps" not in sys.argv:
            args.steps = 16 if cache else 64
        if "--warmup" not in sys.argv:
            args.warmup = 8 if cache else 4
    t_build = time.time()
    if cache:
        dm = CachedModel(c, seed=args.seed, n_layers=args.layers, capacity=args.cache_slots,
                         n_host=args.host_blocks, shared_alias=True,
                         bias_offset=synthdata.zipf_bias_offset(c["n_routed_experts"], args.seed,
                                                                amplitude=args.zipf_amp))
        dm.ctx.cache_set_speculation(args.spec)
    elif batched:
        args.layers = 1
        if "--steps" not in sys.argv:
            args.steps = 20
        if "--warmup" not in sys.argv:
            args.warmup = 3
        zipf_off = synthdata.zipf_bias_offset(c["n_routed_experts"], args.seed, amplitude=args.zipf_amp)
        dm = DeviceModel(c, seed=args.seed, n_layers=1, bias_offset=zipf_off)
    else:
        dm = DeviceModel(c, seed=args.seed, n_layers=args.layers, shared_mxfp4=sh4)
    dm.ctx.set_schedule(moe.SCHED_FUSED if args.sched == "fused" else moe.SCHED_PHASED)
    dm.ctx.set_taps(False)  # the shared-expert output tap is a test hook
    n_h = 64
    hs = np.stack([synthdata.hidden_state(H, 5000 + i) for i in range(n_h)])
    d_hs = hip.DeviceBuffer.from_array(hs)
    d_out = hip.DeviceBuffer(4 * H * args.layers)
    stream = hip.Stream()
    build_s = time.time() - t_build

    d_h, d_tmp = hip.DeviceBuffer(4 * H), hip.DeviceBuffer(4 * H)

    if batched:
        T = args.tokens
        hb = np.stack([synthdata.hidden_state(H, 7000 + (t % 256)) for t in range(T)])
        d_hb = hip.DeviceBuffer.from_array(hb)
        d_ob = hip.DeviceBuffer(4 * H * T)

    def step(i):
        if batched:
            if args.noalloc:
                dm.ctx.run_moe_batched_noalloc(0, T, d_hb.ptr, None, d_ob.ptr, stream.handle)
            else:
                dm.ctx.run_moe_batched(0, T, d_hb.ptr, None, d_ob.ptr, stream.handle)
            return
        if chain:  # one token: its own start state, then h <- h + moe(h) through every layer
            hip.copy_d2d(d_h.ptr, d_hs.ptr + 4 * H * (i % n_h), 4 * H, stream.handle)
            dm.ctx.run_chain(0, args.layers, d_h.ptr, d_tmp.ptr, stream.handle)
            return
        l = i % args.layers
        dm.ctx.run_moe(l, d_hs.ptr + 4 * H * (i % n_h), d_out.ptr + 4 * H * l, stream.handle)

    def measure():
        for i in range(args.warmup):
            step(i)
        dm.ctx.check_error(stream.handle)
        hip.synchronize()
        if cache:
            dm.ctx.cache_reset_stats()
        e0, e1 = hip.Event(), hip.Event()
        e0.record(stream)
        for i in range(args.steps):
            step(args.warmup + i)
        e1.record(stream)
        e1.synchronize()
        ms_ = e0.elapsed_ms(e1)
        dm.ctx.check_error(stream.handle)
        return ms_, (dm.ctx.cache_stats() if cache else None)

    layers_per_step = args.layers if chain else 1
    policies = [p.strip() for p in args.policies.split(",") if p.strip()] if cache else ["-"]
    pinned = []
    if cache and args.pin_top > 0:
        # profile pass: the warm-up tokens layer by layer, the routed keys read back
        from collections import Counter
        E_, K_ = c["n_routed_experts"], c["n_experts_per_tok"]
        cnt = Counter()
        for i in range(args.warmup):
            hip.copy_d2d(d_h.ptr, d_hs.ptr + 4 * H * (i % n_h), 4 * H, stream.handle)
            cur, nxt = d_h, d_tmp
            for l in range(args.layers):
                dm.ctx.run_moe_residual(l, cur.ptr, cur.ptr, nxt.ptr, stream.handle)
                stream.synchronize()
                for e in hip.download_ptr(dm.ctx.taps()["topk_idx"], np.int32, K_):
                    cnt[l * E_ + int(e)] += 1
                cur, nxt = nxt, cur
        pinned = [k for k, _ in cnt.most_common(args.pin_top)]
        for k in pinned:
            dm.ctx.cache_pin(k // E_, k % E_)
    per_policy = {}
    for pol in policies:
        if cache:
            dm.ctx.cache_set_policy(pol)
        ms_p, st_p = measure()
        per_policy[pol] = (ms_p, st_p)
    ms, cstats = per_policy[policies[0]]
    replay = None
    if cache:
        # the request trace of the measured tokens (warm-up + timed, the same
        # start states), recorded layer by layer through the taps, replayed
        # through every policy and through Belady's offline bound; hit rates
        # over the timed tokens, as measured
        E_, K_ = c["n_routed_experts"], c["n_experts_per_tok"]
        dm.ctx.cache_set_policy(policies[0])
        trace = []
        for i in range(args.warmup + args.steps):
            hip.copy_d2d(d_h.ptr, d_hs.ptr + 4 * H * (i % n_h), 4 * H, stream.handle)
            cur, nxt = d_h, d_tmp
            for l in range(args.layers):
                dm.ctx.run_moe_residual(l, cur.ptr, cur.ptr, nxt.ptr, stream.handle)
                stream.synchronize()
                trace += [l * E_ + int(e) for e in hip.download_ptr(dm.ctx.taps()["topk_idx"], np.int32, K_)]
                cur, nxt = nxt, cur
        dm.ctx.check_error(stream.handle)
        t0 = args.warmup * args.layers * K_
        replay = {}
        for pol in ["lru", "lfu", "slru", "2q", "tinylfu", "belady", "belady_bypass"]:
            out = moe.policy_replay(pol, args.cache_slots, trace, K_, pinned=pinned if "belady" not in pol else ())[0]
            timed = out[t0:]
            h_ = int((timed == 1).sum())
            m_ = int(((timed == 0) | (timed == 3)).sum())
            replay[pol] = round(h_ / max(1, h_ + m_), 4)
    us_per_layer = ms * 1e3 / args.steps / layers_per_step

    if args.calib_copy_mb > 0:
        nb = args.calib_copy_mb << 20
        src, dst = hip.DeviceBuffer(nb), hip.DeviceBuffer(nb)
        hip.copy_d2d(dst.ptr, src.ptr, nb, stream.handle)
        stream.synchronize()
        src.free()
        dst.free()

    nbytes = algorithmic_bytes(c, sh4)
    if batched:  # the experts this batch used (each read once), shared, router, T input/output rows
        cnt = dm.ctx.batched_counts()
        H_, I_ = c["hidden"], c["moe_inter"]
        expert = 3 * I_ * H_ // 2 + 3 * I_ * H_ // 32
        uniq = int((cnt > 0).sum())
        nbytes = uniq * expert + 3 * I_ * c["n_shared"] * H_ * 2 + c["n_routed_experts"] * H_ * 2 + \
            c["n_routed_experts"] * 4 + 2 * H_ * 4 * args.tokens
    achieved = nbytes / (us_per_layer * 1e-6) / 1e9
    traffic = None
    if args.workload in ("layer", "chain") and not sh4 and os.path.exists(args.traffic_json):
        try:
            traffic = json.load(open(args.traffic_json)).get("hbm_bytes_per_layer")
        except Exception:
            traffic = None

    cpu = None
    if args.cpu_sample > 0 and not sh4:  # the CPU sample is the bf16-shared layer
        phys, logical = host_cores()
        ncores = min(phys, 16)  # physical cores, at most the box's CPU share for one GPU
        if batched:
            us_all, text = cpu_baseline_batched(c, args.seed, hb, zipf_off, ncores)
            us_one, _ = cpu_baseline_batched(c, args.seed, hb, zipf_off, 1)
            unit = "us/call"
        else:
            us_all, n_all = cpu_baseline(c, args.seed, args.cpu_sample, ncores)
            us_one, n_one = cpu_baseline(c, args.seed, args.cpu_sample, 1)
            unit = "us/layer"
            text = (f"numpy oracle (dequant to f32 + OpenBLAS matvecs) on {n_all} config-1 layers after one "
                    f"warm-up, median; router+8 experts+shared; expert bytes pre-generated"
                    + ("; a chain token is 24 such layers (extrapolated x24)" if chain else ""))
        cpu = {"value": round(us_all, 1), "unit": unit, "cores": ncores, "kind": "port", "sample": text,
               "host_physical_cores": phys, "host_logical_cpus": logical,
               "value_1thread": round(us_one, 1), "gpu_speedup": round(us_all / us_per_layer, 1)}

    line = {
        "metric": "us_per_moe_decode_layer",
        "value": round(us_per_layer, 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(us_per_layer * layers_per_step / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("mxfp4/bf16 weights, f32 activations and accumulation (bf16 MFMA on three exact bf16 pieces "
                  "of each f32 activation); the cross-work-group partial sums are exchanged as f32 rounded to "
                  "21 stored mantissa bits" if not batched else
                  "mxfp4/bf16 weights, f32 activations and accumulation (bf16 MFMA on three exact bf16 pieces "
                  "of each f32 activation)"),
        "data": "synthetic",
        "config": {"workload": (f"config3: one GLM MoE layer over {args.tokens} tokens (batched"
                                f"{', allocation-free entry point' if args.noalloc else ''})" if batched else
                                f"config4: {args.layers} GLM MoE layers behind a {args.cache_slots}-slot HBM expert "
                                f"cache, misses from pinned host memory, bs=1" if cache else
                                f"config2: chain of {args.layers} resident GLM MoE decode layers, bs=1, "
                                f"h <- h + moe(h)" if chain else "config1: one GLM MoE decode layer, bs=1"),
                   "hidden": H, "moe_inter": c["moe_inter"], "n_routed_experts": c["n_routed_experts"],
                   "n_experts_per_tok": c["n_experts_per_tok"],
                   "shared": ("mxfp4" if sh4 else "bf16") + " inter 2048",
                   ("chain_layers" if chain else "rotating_layers"): args.layers, "schedule": args.sched,
                   "global_batch": args.tokens if batched else 1},
        "tokens_per_s": round(1e6 / (us_per_layer * layers_per_step) * (args.tokens if batched else 1), 2),
        "tokens_per_s_per_layer": round(1e6 / us_per_layer, 1),
        "achieved_GBps": round(achieved, 1),
        "pct_of_hbm_peak": round(100 * achieved / PEAK_HBM_GBPS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_HBM_GBPS, 4), "traffic": traffic,
                     "traffic_source": (f"stored figure, not measured in this run: {os.path.relpath(args.traffic_json, ROOT)} "
                                        "(rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of this bench command, "
                                        "scaled by a copy-kernel calibration)") if traffic is not None else None,
                     "algorithmic_bytes": nbytes,
                     "kernel": ("whole batched call (bup_kernel + bdown_kernel dominate)" if batched else
                                f"moe_chain_kernel ({args.layers} layers per launch; per layer)"
                                if args.workload == "chain" and args.sched == "fused" else "moe_decode_kernel")},
        "cpu_baseline": cpu,
        **({"batched": {"tokens": args.tokens, "unique_experts": uniq, "max_tokens_per_expert": int(cnt.max()),
                        "zipf": {"s": 1.1, "amplitude": args.zipf_amp}}} if batched else {}),
        **({"cache": {"hit_rate": round(cstats["hits"] / max(1, cstats["hits"] + cstats["misses"]), 4),
                      "hits": cstats["hits"], "misses": cstats["misses"], "evictions": cstats["evictions"],
                      "speculation": args.spec, "spec_requests": cstats["spec_requests"],
                      "spec_copies": cstats["spec_copies"], "spec_hits": cstats["spec_hits"],
                      "h2d_GB": round(cstats["bytes_h2d"] / 1e9, 3),
                      "h2d_GBps": round(cstats["bytes_h2d"] / (ms * 1e-3) / 1e9, 2),
                      "host_blocks": args.host_blocks, "slots": args.cache_slots, "policy": policies[0],
                      "bypassed": cstats["bypassed"], "pinned": len(pinned),
                      "policies": {pol: {"hit_rate": round(st["hits"] / max(1, st["hits"] + st["misses"]), 4),
                                         "us_per_layer": round(m * 1e3 / args.steps / layers_per_step, 1),
                                         "tokens_per_s": round(1e6 / (m * 1e3 / args.steps), 3),
                                         "bypassed": st["bypassed"], "h2d_GB": round(st["bytes_h2d"] / 1e9, 3)}
                                   for pol, (m, st) in per_policy.items()},
                      "replay_hit_rate": replay,
                      "replay_note": "the timed tokens' request trace (recorded on the GPU) replayed through each "
                                     "policy (pinned keys as measured) and Belady's offline optimum of plain paging "
                                     "without / with bypass (an upper bound for every policy)",
                      "zipf": {"s": 1.1, "amplitude": args.zipf_amp}}} if cache else {}),
        "build_s": round(build_s, 1),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
