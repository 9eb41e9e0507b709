"""Synthetic workloads of the five benchmark configurations.

Every tensor is drawn from a counter-based SplitMix64 stream identified by
(seed, tag), so the GPU generator (q38m_synth_fill) and the CPU
restatement produce identical bytes.  Distributions:

  hidden states   bf16(N(0,1))                       tag 1 (+ layer offset)
  router logits   fp32 N(0,1) + log-popularity bias  tag 2 (+ layer offset)
  W4 group-32     int4 U[-8,7], fp16 |N(0,0.02)|      scale stream tag+1
  W8 per-channel  int8 U[-127,127], fp16 |N(0,0.002)| scale stream tag+1
                  (BASELINE gives no W8 scale distribution; 0.002 keeps the
                  dequantised W8 weights at the W4 weights' magnitude)

Zipf popularity: p_e = rank(e)^-s / sum, rank a seeded permutation of the
experts (Fisher-Yates over SplitMix64); the bias log(p_e) is added to the
N(0,1) logits.
"""
import math

HIDDEN = 2048
INTER = 512
EXPERTS = 512
TOPK = 10

W4 = ("w4", 4, 32, 0.02)
W8 = ("w8", 8, 0, 0.002)

MASK64 = (1 << 64) - 1
GAMMA = 0x9E3779B97F4A7C15


def _mix64(z):
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9 & MASK64
    z = (z ^ (z >> 27)) * 0x94D049BB133111EB & MASK64
    return z ^ (z >> 31)


def rand64(seed, tag, counter):
    base = _mix64((seed + GAMMA * (tag + 1)) & MASK64)
    return _mix64((base + GAMMA * (counter + 1)) & MASK64)


def zipf_bias(seed, tag, s, experts=EXPERTS):
    """log-popularity bias (float list) for Zipf exponent s."""
    perm = list(range(experts))
    for i in range(experts - 1, 0, -1):
        j = (rand64(seed, tag, i) >> 32) * (i + 1) >> 32
        perm[i], perm[j] = perm[j], perm[i]
    weights = [(r + 1) ** (-s) for r in range(experts)]
    total = sum(weights)
    bias = [0.0] * experts
    for rank, e in enumerate(perm):
        bias[e] = math.log(weights[rank] / total)
    return bias


def layer_tags(layer):
    """(gate_up tag, down tag, hidden tag, logits tag) of one layer."""
    base = 1000 + 10 * layer
    return base, base + 4, 1 + 100 * layer, 2 + 100 * layer


def layer_policy(config, layer):
    """(gate_up format, down format) of a layer."""
    if config == 1:
        return W4, W4
    if config == 5:
        return (W4, W4) if layer % 2 == 0 else (W4, W8)
    return W4, W8


CONFIGS = {
    1: {"name": "config1: 64-token MoE layer, all-W4 g32, N(0,1) logits",
        "tokens": 64, "layers": 1, "zipf": None, "seed": 1},
    2: {"name": "config2: 512-token prefill slab, W4 g32 gate/up + W8 per-channel down",
        "tokens": 512, "layers": 1, "zipf": None, "seed": 2},
    3: {"name": "config3: batch-1 decode through 48 MoE layers, W4 g32 gate/up + W8 down",
        "tokens": 1, "layers": 48, "zipf": None, "seed": 3},
    4: {"name": "config4: 4096-token chunk, W4/W8 mixed, Zipf s=1.1 routing",
        "tokens": 4096, "layers": 1, "zipf": 1.1, "seed": 4},
    5: {"name": "config5: 48-layer stack, 32768 tokens as 64 slabs, alternating policy, "
                "Zipf s=0.8",
        "tokens": 32768, "layers": 48, "zipf": 0.8, "seed": 5},
}


def bias_for(config, layer):
    spec = CONFIGS[config]
    if spec["zipf"] is None:
        return None
    return zipf_bias(spec["seed"], 50000 + layer, spec["zipf"])


def algorithmic_bytes_per_expert(gate_up_fmt, down_fmt, hidden=HIDDEN, inter=INTER):
    """Packed weight + scale bytes of one expert (both projections)."""
    def nbytes(fmt, rows, cols):
        _, bits, group, _ = fmt
        data = rows * cols * bits // 8
        scales = (rows * cols // group if group else rows) * 2
        return data + scales
    return nbytes(gate_up_fmt, 2 * inter, hidden) + nbytes(down_fmt, hidden, inter)


def ops_per_route(hidden=HIDDEN, inter=INTER):
    return 2 * (2 * inter * hidden + hidden * inter)
