"""Synthetic inputs of the benchmark configs, reproducible on the CPU.

TEST INFRASTRUCTURE: this module (like everything under oracle/) is only
imported by tests/, bench.py's CPU-baseline leg and __graft_entry__.smoke(), as
the checker. The product path never imports it.

Two generators:

* MXFP4 expert blocks come from a counter-based hash so the GPU can fill tens of
  gigabytes on the device (wl_synth_expert, windlass_amd/csrc/synth.hip) and
  the oracle can rebuild just the experts a token was routed to:
      mix32(x)   = lowbias32 (x ^= x>>16; x *= 0x7feb352d; x ^= x>>15;
                              x *= 0x846ca68b; x ^= x>>16)
      key        = mix32(mix32(seed ^ 0x9E3779B9) ^
                         (layer*0x85EBCA6B + expert*0xC2B2AE35 + 0x27D4EB2F))
      salt[r]    = mix32(0x632BE5AB * (r+1)), r = 0..5 (gate_w, gate_s, up_w,
                   up_s, down_w, down_s)
      word(r, i) = mix32(mix32(i ^ salt[r]) ^ key)
      weight byte j = byte j&3 (little-endian) of word(r, j>>2)  -> codes uniform over 16
      scale byte j  = 118 + word(r, j) % 9                       -> E8M0 exponent in [118,126]
* Dense tensors (router weight, bias, shared expert, hidden state) are drawn
  with numpy's default_rng seeded by (seed, layer, tag), rounded to bf16 (RNE)
  where the config says bf16.
"""
import numpy as np

M32 = np.uint32(0xFFFFFFFF)


def mix32(x):
    x = np.asarray(x, dtype=np.uint32)
    with np.errstate(over="ignore"):
        x = x ^ (x >> np.uint32(16))
        x = (x * np.uint32(0x7FEB352D)).astype(np.uint32)
        x = x ^ (x >> np.uint32(15))
        x = (x * np.uint32(0x846CA68B)).astype(np.uint32)
        x = x ^ (x >> np.uint32(16))
    return x


def mix32_int(x):
    return int(mix32(np.uint32(x & 0xFFFFFFFF)))


def synth_key(seed, layer, expert):
    b = (layer * 0x85EBCA6B + expert * 0xC2B2AE35 + 0x27D4EB2F) & 0xFFFFFFFF
    return mix32_int(mix32_int(seed ^ 0x9E3779B9) ^ b)


def salt(r):
    return mix32_int((0x632BE5AB * (r + 1)) & 0xFFFFFFFF)


def _words(key, r, n):
    i = np.arange(n, dtype=np.uint32)
    return mix32(mix32(i ^ np.uint32(salt(r))) ^ np.uint32(key))


def region_bytes(key, r, nbytes):
    """Bytes of region r (0..5) of an expert block."""
    if r % 2 == 0:
        assert nbytes % 4 == 0
        return _words(key, r, nbytes // 4).view(np.uint8).copy()
    return (np.uint32(118) + _words(key, r, nbytes) % np.uint32(9)).astype(np.uint8)


def expert_block(H, I, seed, layer, expert):
    """The six sub-tensors of one packed expert: gate_w [I,H/2], gate_s [I,H/32],
    up_w, up_s, down_w [H,I/2], down_s [H,I/32] (all uint8)."""
    key = synth_key(seed, layer, expert)
    shapes = [(I, H // 2), (I, H // 32), (I, H // 2), (I, H // 32), (H, I // 2), (H, I // 32)]
    return [region_bytes(key, r, a * b).reshape(a, b) for r, (a, b) in enumerate(shapes)]


def expert_block_bytes(H, I, seed, layer, expert):
    """The packed block exactly as it sits in HBM (ExpertLayout order)."""
    return np.concatenate([t.reshape(-1) for t in expert_block(H, I, seed, layer, expert)])


# ---- bf16 ----------------------------------------------------------------------
def f32_to_bf16(x):
    """Round-to-nearest-even fp32 -> bf16 bits (reference f32_to_bf16,
    src/safetensors_io.cuh:239-243)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    return r.astype(np.uint16)


def bf16_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


TAG_ROUTER, TAG_BIAS, TAG_SH_GATE, TAG_SH_UP, TAG_SH_DOWN, TAG_HIDDEN, TAG_LN = 1, 2, 3, 4, 5, 6, 7


def _rng(seed, layer, tag):
    return np.random.default_rng(np.random.SeedSequence([seed, layer, tag]))


def normal_bf16(seed, layer, tag, shape, std):
    x = _rng(seed, layer, tag).standard_normal(size=shape, dtype=np.float32) * np.float32(std)
    return f32_to_bf16(x).reshape(shape)


def dense_layer(H, E, SI, seed, layer):
    """Router weight [E,H] bf16 ~ N(0,0.02), bias [E] f32 ~ N(0,0.01), and the
    shared expert as one bf16 block [gate SI*H | up SI*H | down H*SI] ~ N(0,0.02)."""
    router_w = normal_bf16(seed, layer, TAG_ROUTER, (E, H), 0.02)
    bias = (_rng(seed, layer, TAG_BIAS).standard_normal(size=E, dtype=np.float32)
            * np.float32(0.01)).astype(np.float32)
    sg = normal_bf16(seed, layer, TAG_SH_GATE, (SI, H), 0.02)
    su = normal_bf16(seed, layer, TAG_SH_UP, (SI, H), 0.02)
    sd = normal_bf16(seed, layer, TAG_SH_DOWN, (H, SI), 0.02)
    return {"router_w": router_w, "bias": bias, "sh_gate": sg, "sh_up": su, "sh_down": sd,
            "shared_block": np.concatenate([sg.reshape(-1), su.reshape(-1), sd.reshape(-1)])}


def hidden_state(H, seed, step=0):
    """bf16 N(0,1) hidden state, widened to f32 (the layer input)."""
    return bf16_to_f32(normal_bf16(seed, step, TAG_HIDDEN, (H,), 1.0))


def zipf_bias_offset(E, seed, s=1.1, amplitude=0.05):
    """Zipf(s)-shaped popularity offset for the router bias (configs 3 and 4):
    expert ranked r (random permutation, seeded) gets amplitude * r^-s."""
    perm = np.random.default_rng(np.random.SeedSequence([seed, 0xF00D])).permutation(E)
    off = np.empty(E, dtype=np.float32)
    off[perm] = (np.float32(amplitude) * (np.arange(1, E + 1, dtype=np.float64) ** -s)).astype(np.float32)
    return off
