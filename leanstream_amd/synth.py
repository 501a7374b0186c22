"""Synthetic sparse-MLP workloads (host mirror of the device generator in csrc/synth.hip).

Element i of every stream is mix64(seed + (i + 1) * 0x9E3779B97F4A7C15) (splitmix64),
so host (numpy) and device generation produce identical bytes:
  * packed INT4 weights: the little-endian bytes of the stream (uniform nibbles in [-8, 7]);
  * fp16 scales: lo + (hi - lo) * u, u = (value >> 11) * 2^-53, rounded to fp16;
  * fp16 / bf16 activations: standard normal by the Box-Muller transform of elements 2i and
    2i + 1, rounded to fp16 / bf16 (normal_f64 states the arithmetic);
  * group scores: the same normal in fp32.

Workloads named here are the layer shapes this library is measured on (d_model, d_ffn,
64-neuron groups, active fraction k = floor(frac * groups + 0.5)).
"""
from dataclasses import dataclass, field

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

SEED_X, SEED_W, SEED_S, SEED_SCORE, SEED_ORDER = 1, 2, 3, 4, 5


def stream(seed, index):
    index = np.asarray(index, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (index + np.uint64(1)) * GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def unit(seed, index):
    return (stream(seed, index) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)


def fill_bytes(n, seed):
    words = stream(seed, np.arange((n + 7) // 8, dtype=np.uint64))
    return words.astype("<u8").view(np.uint8)[:n].copy()


def uniform_f16(n, seed, lo, hi):
    return (lo + (hi - lo) * unit(seed, np.arange(n, dtype=np.uint64))).astype(np.float16)


def _ln_unit(u):
    """ln(u) for u in (0, 1] with IEEE +, -, *, / only (no library log): u = m 2^e with m in
    [sqrt(1/2), sqrt(2)), ln m = 2 atanh(t), t = (m - 1) / (m + 1), series to t^25 in Horner form."""
    m, e = np.frexp(u)
    low = m < 0.7071067811865476
    m = np.where(low, m * 2.0, m)
    e = np.where(low, e - 1, e).astype(np.float64)
    t = (m - 1.0) / (m + 1.0)
    t2 = t * t
    p = np.full_like(t, 1.0 / 25.0)
    for k in range(11, -1, -1):
        p = p * t2 + 1.0 / (2 * k + 1)
    return e * 0.6931471805599453 + 2.0 * t * p


def _cos_turns(v):
    """cos(2 pi v) for v in [0, 1) with IEEE +, -, *, / only: quadrant q = floor(4 v) (exact),
    x = (4 v - q) pi / 2, Taylor series of cos x and sin x to x^22 / x^23 in Horner form."""
    w = v * 4.0
    q = np.floor(w)
    x = (w - q) * 1.5707963267948966
    x2 = x * x
    c = np.full_like(x, _COS_C[-1])
    s = np.full_like(x, _SIN_C[-1])
    for k in range(len(_COS_C) - 2, -1, -1):
        c = c * x2 + _COS_C[k]
        s = s * x2 + _SIN_C[k]
    s = s * x
    return np.where(q == 0, c, np.where(q == 1, -s, np.where(q == 2, -c, s)))


def _taylor(first):
    out, f, k = [], 1.0, first
    for _ in range(12):
        out.append(f)
        f = -f / ((k + 1) * (k + 2))
        k += 2
    return out


_COS_C = _taylor(0)   # (-1)^k / (2k)!     as the sequence of divisions above gives them
_SIN_C = _taylor(1)   # (-1)^k / (2k + 1)!


def normal_f64(n, seed):
    """Standard normal values: Box-Muller of u1 = ((v(2i) >> 11) + 1) 2^-53 in (0, 1] and
    u2 = (v(2i+1) >> 11) 2^-53 in [0, 1): sqrt(-2 ln u1) cos(2 pi u2). Every step is an IEEE
    double operation (frexp, +, -, *, /, sqrt) in a fixed order, so the C oracle and the device
    generator compute the same doubles."""
    i = np.arange(n, dtype=np.uint64) * np.uint64(2)
    u1 = ((stream(seed, i) >> np.uint64(11)) + np.uint64(1)).astype(np.float64) * (2.0 ** -53)
    u2 = unit(seed, i + np.uint64(1))
    return np.sqrt(-2.0 * _ln_unit(u1)) * _cos_turns(u2)


def normal_f16(n, seed):
    return normal_f64(n, seed).astype(np.float16)


def f64_to_bf16_bits(v):
    """Round-to-nearest-even double -> bfloat16 bits (the device generator's conversion)."""
    b = np.asarray(v, dtype=np.float64).view(np.uint64)
    sign = (b >> np.uint64(48)) & np.uint64(0x8000)
    exp = ((b >> np.uint64(52)) & np.uint64(0x7FF)).astype(np.int64)
    mant = b & np.uint64(0xFFFFFFFFFFFFF)
    e = exp - 1023 + 127
    m = (mant >> np.uint64(45)).astype(np.int64)
    rem = mant & np.uint64((1 << 45) - 1)
    half = np.uint64(1 << 44)
    m = m + ((rem > half) | ((rem == half) & (m % 2 == 1))).astype(np.int64)
    carry = m == 128
    m = np.where(carry, 0, m)
    e = e + carry
    out = sign.astype(np.int64) | (np.clip(e, 0, 255) << 7) | m
    out = np.where(e >= 255, sign.astype(np.int64) | 0x7F80, out)
    out = np.where((exp == 0) | (e <= 0), sign.astype(np.int64), out)
    return out.astype(np.uint16)


def normal_bf16(n, seed):
    """bfloat16 bits of the normal stream."""
    return f64_to_bf16_bits(normal_f64(n, seed))


def bf16_to_f16(bits):
    """bf16 bits -> fp16 (through fp32, round to nearest even): what the dense kernels feed
    the matrix cores; exact unless |x| < 2^-17."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32).astype(np.float16)


def permutation(n, seed):
    """Fisher-Yates driven by the stream: j = value(i) mod (i + 1), i from n-1 down."""
    perm = np.arange(n, dtype=np.int64)
    vals = stream(seed, np.arange(n, dtype=np.uint64))
    for i in range(n - 1, 0, -1):
        j = int(vals[i] % np.uint64(i + 1))
        perm[i], perm[j] = perm[j], perm[i]
    return perm


def rank_top_k(scores, k):
    """Top-k ids by (score descending, id ascending) (predictor_cpu.cpp:192-201)."""
    scores = np.asarray(scores, dtype=np.float32)
    order = np.lexsort((np.arange(len(scores)), -scores.astype(np.float64)))
    return order[:k].astype(np.int64)


@dataclass(frozen=True)
class LayerConfig:
    name: str
    width: int               # d_model
    ffn: int                 # d_ffn
    active_frac: float
    group_size: int = 64
    batch: int = 1
    scale_lo: float = 0.005
    scale_hi: float = 0.02
    selection: str = "ranking"   # "ranking" (N(0,1) scores, top-k) | "permutation" | "all"
    seed: int = 0x1EA5_5EED
    x_dtype: str = "f16"         # "f16" | "bf16" (the dense batched path)

    @property
    def groups(self):
        return self.ffn // self.group_size

    @property
    def active(self):
        return int(np.floor(self.active_frac * self.groups + 0.5))

    @property
    def group_bytes(self):
        return self.group_size * 3 * self.width // 2

    @property
    def scale_words(self):
        """fp16 scales per group: G neurons x 3 projections x d/128 blocks."""
        return self.group_size * 3 * (self.width // 128)

    def sub_seed(self, tag):
        return (self.seed * 0x100000001B3 + tag) & 0xFFFFFFFFFFFFFFFF

    def algorithmic_bytes(self):
        """INT4 weights + fp16 scales of the active groups + x in + y out."""
        k, G, d = self.active, self.group_size, self.width
        return k * G * (3 * d // 2) + k * G * 3 * (d // 128) * 2 + 2 * self.batch * d * 2


CONFIGS = {
    "c1": LayerConfig("sparse_int4_mlp_d1024_f4096_g64_a25", 1024, 4096, 0.25, selection="permutation",
                      seed=0xC1),
    "c2": LayerConfig("ministral8b_sparse_int4_mlp_d4096_f12288_a30_b1", 4096, 12288, 0.30, seed=0xC2),
    "c4": LayerConfig("llama70b_sparse_int4_mlp_d8192_f28672_a20_b1", 8192, 28672, 0.20, scale_lo=0.003,
                      scale_hi=0.015, seed=0xC4),
    # batch 4: the same weights and active groups as the batch-1 entries (same seed); x
    # row 0 is their x (the generator is counter-based)
    "c4b4": LayerConfig("llama70b_sparse_int4_mlp_d8192_f28672_a20_b4", 8192, 28672, 0.20, batch=4,
                        scale_lo=0.003, scale_hi=0.015, seed=0xC4),
    "c1b4": LayerConfig("sparse_int4_mlp_d1024_f4096_g64_a25_b4", 1024, 4096, 0.25, batch=4,
                        selection="permutation", seed=0xC1),
    # dense batched fallback: every group active, batch 32, bf16 x (matrix-core path)
    "c5": LayerConfig("dense_int4_mlp_d4096_f14336_g64_b32", 4096, 14336, 1.0, batch=32, selection="all",
                      x_dtype="bf16", seed=0xC5),
    # Ministral-3 8B production geometry: Group2 bundles (2-neuron groups, 7168 groups), 1434
    # active (20%), as LeanStream's Ministral packer lays them out
    "g2": LayerConfig("ministral3_8b_group2_sparse_int4_mlp_d4096_f14336_a20_b1", 4096, 14336, 0.20, group_size=2,
                      seed=0x62),
    # the same path at the d_model 1024 shape, 16 of 64 groups (quick parity case)
    "c1d32": LayerConfig("sparse_int4_mlp_d1024_f4096_g64_a25_b32", 1024, 4096, 0.25, batch=32,
                         selection="permutation", x_dtype="bf16", seed=0xC1),
}


def physical_of(logical, groups):
    """Fixed bijection logical -> physical (storage order differs from predictor ids)."""
    return (np.asarray(logical, dtype=np.int64) * 37 + 11) % groups


def active_groups(cfg):
    """Logical ids of the active groups, in execution (rank / publication) order."""
    if cfg.selection == "all":
        return np.arange(cfg.groups, dtype=np.int64)
    if cfg.selection == "permutation":
        return permutation(cfg.groups, cfg.sub_seed(SEED_SCORE))[: cfg.active]
    scores = normal_f64(cfg.groups, cfg.sub_seed(SEED_SCORE)).astype(np.float32)
    return rank_top_k(scores, cfg.active)


def group_scores(cfg):
    return normal_f64(cfg.groups, cfg.sub_seed(SEED_SCORE)).astype(np.float32)


def ready_order(count, cfg):
    """Publication order of queue descriptors (a seeded permutation of 0..count-1)."""
    return permutation(count, cfg.sub_seed(SEED_ORDER))


@dataclass
class HostLayer:
    """A whole layer in host memory: cache arena in physical order, scales, x."""

    cfg: LayerConfig
    cache: np.ndarray = field(repr=False)    # uint8 [groups * group_bytes]
    scales: np.ndarray = field(repr=False)   # float16 [groups * scale_words]
    x: np.ndarray = field(repr=False)        # float16 [batch * width] (bf16 x: its exact fp16 value)


def host_layer(cfg):
    cache = fill_bytes(cfg.groups * cfg.group_bytes, cfg.sub_seed(SEED_W))
    scales = uniform_f16(cfg.groups * cfg.scale_words, cfg.sub_seed(SEED_S), cfg.scale_lo, cfg.scale_hi)
    if cfg.x_dtype == "bf16":
        x = bf16_to_f16(normal_bf16(cfg.batch * cfg.width, cfg.sub_seed(SEED_X)))
    else:
        x = normal_f16(cfg.batch * cfg.width, cfg.sub_seed(SEED_X))
    return HostLayer(cfg, cache, scales, x)


def descriptors(cfg, logical, source_kind=0, dest_base=0):
    """ExecDesc rows (uint32 [n, 5]) for the given logical ids: source slot and scale
    row are the physical group; destinations are dest_base + position."""
    logical = np.asarray(logical, dtype=np.int64)
    phys = physical_of(logical, cfg.groups)
    out = np.zeros((len(logical), 5), dtype=np.uint32)
    out[:, 0] = logical
    out[:, 1] = phys
    out[:, 2] = phys
    out[:, 3] = dest_base + np.arange(len(logical))
    out[:, 4] = source_kind
    return out


# ---------------------------------------------------------------- streaming decode step
SEED_ARRIVAL = 6


@dataclass(frozen=True)
class StreamConfig:
    """A decode step of `layers` sparse MLP layers of one shape whose active groups are
    staged from pinned host memory. Layer l has its own weights, scales and N(0,1) group
    scores (seed derived from `seed` and l); x is shared. In rank order, group i's bytes
    reach the pinned store at the sum of i+1 exponential gaps of mean `arrival_mean_ns`."""

    name: str
    layer: LayerConfig
    layers: int = 36
    arrival_mean_ns: float = 5000.0
    seed: int = 0xC3

    def layer_config(self, l):
        return LayerConfig(f"{self.layer.name}_l{l}", self.layer.width, self.layer.ffn, self.layer.active_frac,
                           self.layer.group_size, self.layer.batch, self.layer.scale_lo, self.layer.scale_hi,
                           "ranking", (self.seed * 1000003 + l) & 0xFFFFFFFFFFFFFFFF)

    def x_config(self):
        return self.layer_config(0)

    def arrivals(self, l, rank):
        """ns after the layer's begin at which each logical group may be copied (0 for
        groups outside `rank`)."""
        out = np.zeros(self.layer.groups, dtype=np.uint64)
        if self.arrival_mean_ns <= 0:
            return out
        u = unit(self.layer_config(l).sub_seed(SEED_ARRIVAL), np.arange(len(rank), dtype=np.uint64))
        gaps = -self.arrival_mean_ns * np.log1p(-u)
        out[np.asarray(rank, dtype=np.int64)] = np.floor(np.cumsum(gaps) + 0.5).astype(np.uint64)
        return out


STREAMS = {
    "c3": StreamConfig("streaming_decode_36x_sparse_int4_mlp_d1024_f4096_g64_a25_b1",
                       LayerConfig("sparse_int4_mlp_d1024_f4096_g64_a25", 1024, 4096, 0.25)),
}


def stream_rank(sc, l):
    """Active groups of layer l in rank order (top-k of its N(0,1) scores)."""
    return active_groups(sc.layer_config(l))
