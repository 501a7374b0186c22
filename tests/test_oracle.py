"""Pins the CPU oracle (oracle/oracle.c) before the GPU results are checked against it.

Checks, chosen so that a plausible oracle mistake fails one of them:
  * generator: numpy mirror == C oracle, bit for bit (catches seed/counter/rounding slips);
  * fp16 conversions: exhaustive / edge cases against numpy's IEEE conversions;
  * closed-form known answers from the reference's own tests
    (tests/persistent_mlp_test.cu:52-56, tests/triton_smoke.py:74-77,
     examples/end_to_end/main.cu:75-79, docs/custom_triton.md numerical example);
  * an independent float64 brute force built from the packing format
    (examples/ministral/pack/int4_format.py:21-28 dequantize semantics) on tiny shapes;
  * the ranking comparator against examples/predictor/main.cpp:11 and brute force with ties.
"""
import numpy as np
import pytest

import oracle
from leanstream_amd import synth

f16 = np.float16


def half(v):
    return float(np.float16(v))


# ---------------------------------------------------------------- generator
@pytest.mark.parametrize("n,seed", [(1, 0), (7, 1), (1000, 7), (4097, 0xC2)])
def test_generator_matches_numpy_mirror(n, seed):
    assert np.array_equal(synth.fill_bytes(n, seed), oracle.fill_bytes(n, seed))
    a = synth.uniform_f16(n, seed, 0.005, 0.02).view(np.uint16)
    b = oracle.fill_uniform_f16(n, seed, 0.005, 0.02).view(np.uint16)
    assert np.array_equal(a, b)
    a = synth.normal_f16(n, seed).view(np.uint16)
    b = oracle.fill_normal_f16(n, seed).view(np.uint16)
    assert np.array_equal(a, b)


def test_generator_statistics():
    x = synth.normal_f16(200000, 99).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    # normal, not a bounded approximation: fourth moment 3, tails beyond 4 sigma at 6.3e-5
    z = synth.normal_f64(400000, 99)
    assert abs(((z - z.mean()) ** 4).mean() / z.var() ** 2 - 3.0) < 0.05
    assert 3.5e-5 < (np.abs(z) > 4.0).mean() < 9.5e-5
    s = synth.uniform_f16(100000, 5, 0.005, 0.02).astype(np.float64)
    assert s.min() >= 0.005 - 1e-5 and s.max() <= 0.02 + 1e-5
    b = synth.fill_bytes(1 << 16, 3)
    nib = np.concatenate([b & 15, b >> 4])
    counts = np.bincount(nib, minlength=16)
    assert counts.min() > 0.9 * len(nib) / 16


def test_normal_generator_is_box_muller():
    """The series ln / cos of the generator against the library functions, and the whole
    transform against the textbook sqrt(-2 ln u1) cos(2 pi u2) on the same uniforms."""
    u = np.concatenate([np.linspace(0.0, 1.0, 20001)[1:], 2.0 ** -np.arange(1.0, 54.0), [2.0 ** -53]])
    assert np.max(np.abs(synth._ln_unit(u) - np.log(u))) < 1e-14
    v = np.linspace(0.0, 1.0, 20000, endpoint=False)
    assert np.max(np.abs(synth._cos_turns(v) - np.cos(2.0 * np.pi * v))) < 1e-15
    n, seed = 5000, 0x5EED
    i = np.arange(n, dtype=np.uint64) * np.uint64(2)
    u1 = ((synth.stream(seed, i) >> np.uint64(11)) + np.uint64(1)).astype(np.float64) * 2.0 ** -53
    u2 = synth.unit(seed, i + np.uint64(1))
    textbook = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    assert np.max(np.abs(synth.normal_f64(n, seed) - textbook)) < 1e-12
    # a planted mistake (sin for cos) is caught by the same comparison
    assert np.max(np.abs(np.sqrt(-2.0 * np.log(u1)) * np.sin(2.0 * np.pi * u2) - textbook)) > 0.5


# ---------------------------------------------------------------- fp16
def test_f16_to_f32_exhaustive():
    lib = oracle.lib()
    bits = np.arange(1 << 16, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([lib.ora_f16_to_f32(int(b)) for b in bits[::7]], dtype=np.float32)
    r = ref[::7]
    same = (got == r) | (np.isnan(got) & np.isnan(r))
    assert same.all()


def test_f32_and_f64_to_f16_round_to_nearest_even():
    lib = oracle.lib()
    rng = np.random.default_rng(0)
    vals = np.concatenate([rng.standard_normal(3000) * 10.0 ** rng.integers(-8, 5, 3000),
                           [0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e-8, 2.0 ** -25, 2.0 ** -24, 3 * 2.0 ** -26,
                            1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, np.inf, -np.inf]])
    for v in vals:
        assert lib.ora_f64_to_f16(float(v)) == np.float16(v).view(np.uint16), v
        v32 = np.float32(v)
        assert lib.ora_f32_to_f16(float(v32)) == np.float16(v32).view(np.uint16), v32


# ---------------------------------------------------------------- closed forms
def _kat_layer(H, G, count, byte, scale=0.05, xv=0.1):
    """count+1 groups of identical bytes, all executed, dest slots 0..count."""
    all_ = count + 1
    cache = np.full(all_ * G * 3 * H // 2, byte, dtype=np.uint8)
    scales = np.full(all_ * G * 3 * H // 128, scale, dtype=f16)
    x = np.full(H, xv, dtype=f16)
    descs = np.array([[i, i, i, i, i % 2] for i in range(all_)], dtype=np.uint32)
    return oracle.layer(descs, all_, cache, scales, x, H, G, staging=cache)


@pytest.mark.parametrize("H,G,count", [(256, 2, 0), (256, 2, 1), (256, 2, 16), (256, 2, 37), (512, 2, 3)])
@pytest.mark.parametrize("byte,q", [(0x11, 1), (0xFF, -1)])
def test_closed_form_known_answer(H, G, count, byte, q):
    # tests/persistent_mlp_test.cu:52-56: gate = fp16(H*x*s*q), act = fp16(fp16(silu(gate))*gate),
    # y = fp16(N*G*act*s*q) with N executed groups (tolerance .002).
    out = _kat_layer(H, G, count, byte)
    s, x = half(0.05), half(0.1)
    gate = half(H * x * s * q)
    act = half(half(gate / (1 + np.exp(-gate))) * gate)
    expected = half((count + 1) * G * act * s * q)
    assert np.all(np.abs(out["y16"].astype(np.float32) - expected) < 0.002)
    assert np.allclose(out["h"], act)


def test_custom_triton_numerical_example():
    # docs/custom_triton.md: H=512, INT4=1, scale .05, x .1 -> gate approximately 2.56 before activation.
    out = _kat_layer(512, 2, 0, 0x11)
    gate = half(512 * half(0.1) * half(0.05))
    assert abs(gate - 2.56) < 0.01
    act = half(half(gate / (1 + np.exp(-gate))) * gate)
    assert np.allclose(out["h"], act)


# ---------------------------------------------------------------- float64 brute force
def _dequant(packed, scales_row, width):
    """int4_format.py:21-28: low nibble = even coordinate, two's complement,
    fp32 multiply then fp16."""
    q = np.empty(packed.size * 2, dtype=np.int8)
    q[0::2] = (packed & 15).astype(np.int8)
    q[1::2] = (packed >> 4).astype(np.int8)
    q[q >= 8] -= 16
    s = np.repeat(scales_row.astype(np.float32), 128)
    return (q.astype(np.float32) * s).astype(np.float16).astype(np.float64)


def brute_force(descs, rows, cache, scales, x, width, G, staging=None, swap_nibbles=False):
    staging = cache if staging is None else staging
    gb = G * 3 * width // 2
    partial = np.zeros((rows, width))
    xv = x.astype(np.float64)
    for d in descs:
        arena = staging if d[4] == 1 else cache
        grp = arena[d[2] * gb:(d[2] + 1) * gb].reshape(G, 3, width // 2)
        if swap_nibbles:
            grp = ((grp & 15) << 4) | (grp >> 4)
        sc = scales[d[1] * G * 3 * (width // 128):(d[1] + 1) * G * 3 * (width // 128)].reshape(G, 3, width // 128)
        for n in range(G):
            wg = _dequant(grp[n, 0], sc[n, 0], width)
            wu = _dequant(grp[n, 1], sc[n, 1], width)
            wd = _dequant(grp[n, 2], sc[n, 2], width)
            g = half(wg @ xv)
            u = half(wu @ xv)
            h = half(half(g / (1 + np.exp(-g))) * u)
            partial[d[3]] += h * wd
    return partial.sum(0)


@pytest.mark.parametrize("width,G,groups,seed", [(256, 2, 4, 1), (512, 4, 6, 2), (1024, 8, 3, 3)])
def test_oracle_matches_float64_brute_force(width, G, groups, seed):
    cache = synth.fill_bytes(groups * G * 3 * width // 2, seed)
    staging = synth.fill_bytes(groups * G * 3 * width // 2, seed + 100)
    scales = synth.uniform_f16(groups * G * 3 * (width // 128), seed + 1, 0.005, 0.02)
    x = synth.normal_f16(width, seed + 2)
    perm = synth.permutation(groups, seed + 3)
    descs = np.array([[i, perm[i], (i * 5) % groups, i, i % 2] for i in range(groups)], dtype=np.uint32)
    out = oracle.layer(descs, groups, cache, scales, x, width, G, staging=staging)
    ref = brute_force(descs, groups, cache, scales, x, width, G, staging=staging)
    err = np.abs(out["y32"] - ref)
    assert err.max() <= 1e-4 * max(1.0, np.abs(ref).max())
    # a plausible mistake (nibble order swapped) is far outside that bound
    wrong = brute_force(descs, groups, cache, scales, x, width, G, staging=staging, swap_nibbles=True)
    assert np.abs(wrong - out["y32"]).max() > 100 * max(err.max(), 1e-6)


def test_reduction_is_slot_ordered_fp32():
    rows, width = 5, 256
    rng = np.random.default_rng(4)
    partial = rng.standard_normal((rows, width)).astype(np.float32) * 1e3
    y32 = np.zeros(width, dtype=np.float32)
    y16 = np.zeros(width, dtype=np.uint16)
    oracle.lib().ora_reduce(partial.ctypes.data, rows, width, y32.ctypes.data, y16.ctypes.data)
    acc = np.zeros(width, dtype=np.float32)
    for i in range(rows):
        acc = (acc + partial[i]).astype(np.float32)
    assert np.array_equal(acc, y32)
    assert np.array_equal(acc.astype(np.float16).view(np.uint16), y16)


# ---------------------------------------------------------------- ranking
def test_ranking_known_answer():
    # examples/predictor/main.cpp:11: rows scored by increasing weight -> top-2 ids [3, 2]
    scores = np.array([1.0, 2.0, 3.0, 4.0], dtype=np.float32)
    assert list(oracle.rank(scores, 2)) == [3, 2]


def test_ranking_ties_break_by_id():
    rng = np.random.default_rng(1)
    scores = rng.integers(0, 5, 300).astype(np.float32)
    brute = sorted(range(300), key=lambda i: (-scores[i], i))[:40]
    assert list(oracle.rank(scores, 40)) == brute
    assert list(synth.rank_top_k(scores, 40)) == brute


def test_ranking_rejects_nonfinite():
    with pytest.raises(ValueError):
        oracle.rank(np.array([1.0, np.nan], dtype=np.float32), 1)


def test_f64_to_bf16_round_to_nearest_even():
    """The bf16 conversion of the dense path's x generator: known answers (values checked
    against torch's conversion), then correct rounding against both neighbours on a sample
    of the generator's own values (torch rounds double -> float -> bf16 and can differ at
    the float midpoint; this conversion rounds once)."""
    v = np.array([0.0, 1.0, -1.0, 1.00390625, 1.005859375, 1.0078125, 3.14159, -5.99, 1e-3, 1.001953125])
    want = np.array([0, 16256, 49024, 16256, 16257, 16257, 16457, 49344, 14979, 16256], dtype=np.uint16)
    assert np.array_equal(synth.f64_to_bf16_bits(v), want)
    x = synth.normal_f64(20000, 0x5EED)
    q = synth.f64_to_bf16_bits(x)
    as_f64 = lambda b: (b.astype(np.uint32) << np.uint32(16)).view(np.float32).astype(np.float64)
    val = as_f64(q)
    up, down = as_f64(q + np.uint16(1)), as_f64(q - np.uint16(1))   # neighbours in magnitude
    err = np.abs(val - x)
    assert np.all(err <= np.abs(up - x)) and np.all(err <= np.abs(down - x))
    ties = (err == np.abs(up - x)) | (err == np.abs(down - x))
    assert np.all(q[ties] % 2 == 0)
    # bf16 -> fp16 is exact for these magnitudes
    f16 = synth.bf16_to_f16(q).astype(np.float64)
    big = np.abs(val) >= 2.0 ** -17
    assert np.array_equal(f16[big], val[big])


# ---------------------------------------------------------------------------- epilogue
def test_publish_hidden_closed_forms():
    rng = np.random.default_rng(21)
    y = rng.standard_normal(4096).astype(np.float16)
    r = rng.standard_normal(4096).astype(np.float16)
    z = np.zeros(4096, dtype=np.float16)
    assert np.array_equal(oracle.publish_hidden(z, y).view(np.uint16), y.view(np.uint16))
    assert np.array_equal(oracle.publish_hidden(r, z).view(np.uint16), r.view(np.uint16))
    assert np.array_equal(oracle.publish_hidden(r, y).view(np.uint16), oracle.publish_hidden(y, r).view(np.uint16))
    # the sum of two fp16 values is exact in float64: one rounding of the exact sum (numpy)
    want = (r.astype(np.float64) + y.astype(np.float64)).astype(np.float16)
    assert np.array_equal(oracle.publish_hidden(r, y).view(np.uint16), want.view(np.uint16))


def test_rmsnorm_closed_forms_and_planted_mistake():
    w1 = np.ones(4096, dtype=np.float16)
    # a constant row c: mean(x^2) = c^2, so x / rms = 1 (eps 0), within fp32 rounding of 1/sqrt
    for c in (0.5, -3.0, 1e-2):
        out = oracle.rmsnorm(np.full(4096, c, dtype=np.float16), w1, 0.0).astype(np.float64)
        assert np.all(np.abs(out - np.sign(c)) <= 2.0 ** -10), c
    # eps adds to the mean square, not the sum: c = 1, eps = 3 -> 1 / sqrt(4) = 0.5
    out = oracle.rmsnorm(np.ones(1024, dtype=np.float16), np.ones(1024, dtype=np.float16), 3.0)
    assert np.all(out == np.float16(0.5))
    # brute force in float64 (the fp16 roundings of x / rms and of the weight product)
    rng = np.random.default_rng(5)
    x = rng.standard_normal(4096).astype(np.float16)
    w = rng.uniform(0.5, 1.5, 4096).astype(np.float16)
    xf = x.astype(np.float64)
    inv = 1.0 / np.sqrt(np.mean(xf * xf) + 1e-5)
    want = (w.astype(np.float64) * (xf * inv).astype(np.float16).astype(np.float64)).astype(np.float16)
    got = oracle.rmsnorm(x, w, 1e-5)
    ulps = np.abs(got.view(np.int16).astype(np.int64) - want.view(np.int16).astype(np.int64))
    assert ulps.max() <= 1 and np.count_nonzero(ulps) < 40
    # scaling the weight by 2 scales the output exactly (outside fp16's subnormal range,
    # where rounding is not scale-invariant)
    twice = oracle.rmsnorm(x, (w.astype(np.float32) * 2).astype(np.float16), 1e-5).astype(np.float32)
    normal = np.abs(got.astype(np.float32)) >= 2.0 ** -14
    assert normal.sum() > 4000
    assert np.array_equal(twice[normal], got.astype(np.float32)[normal] * 2)


# ---------------------------------------------------------------- tolerance vs arithmetic
def test_exact_products_leave_the_stated_tolerance_at_c2():
    """Why the kernels form fp16(q*s) per weight (int4_format.py:21-28, streaming_mlp.cu:11-15)
    instead of taking the scale and the nibble bias out of the sums: at the C2 shape
    LeanStream's own per-weight rounding moves y32 further from exact arithmetic than the
    stated max-abs 2e-2, so a kernel computing exact products (a factored dequantisation)
    would fail the tolerance against the oracle, while one that rounds each weight like the
    reference differs only by fp32 summation order. Exact products in float64: g and u of
    every active neuron, its h with the reference's fp16 roundings, y = sum h * (q * s)."""
    cfg = synth.CONFIGS["c2"]
    hl = synth.host_layer(cfg)
    logical = synth.active_groups(cfg)
    rows = synth.descriptors(cfg, logical)
    d, G = cfg.width, cfg.group_size
    ref = oracle.layer(rows, len(rows), hl.cache, hl.scales, hl.x, d, G, threads=8)["y32"].astype(np.float64)
    xv = hl.x.astype(np.float64)
    gb, sw = cfg.group_bytes, G * 3 * (d // 128)
    exact = np.zeros(d)
    rounded = np.zeros(d)
    for row in rows:
        grp = hl.cache[int(row[2]) * gb:(int(row[2]) + 1) * gb].reshape(G, 3, d // 2)
        sc = hl.scales[int(row[1]) * sw:(int(row[1]) + 1) * sw].reshape(G, 3, d // 128)
        q = np.empty((G, 3, d), dtype=np.int8)
        q[..., 0::2] = (grp & 15).astype(np.int8)
        q[..., 1::2] = (grp >> 4).astype(np.int8)
        q[q >= 8] -= 16
        s = np.repeat(sc.astype(np.float32), 128, axis=2)
        for name, w in (("exact", q * s.astype(np.float64)),
                        ("rounded", (q.astype(np.float32) * s).astype(np.float16).astype(np.float64))):
            g = (w[:, 0] @ xv).astype(np.float16).astype(np.float64)
            u = (w[:, 1] @ xv).astype(np.float16).astype(np.float64)
            silu = (g / (1.0 + np.exp(-g))).astype(np.float16).astype(np.float64)
            h = (silu * u).astype(np.float16).astype(np.float64)
            if name == "exact":
                exact += h @ w[:, 2]
            else:
                rounded += h @ w[:, 2]
    rel = lambda a: np.linalg.norm(a - ref) / np.linalg.norm(ref)
    # per-weight rounding: the oracle's arithmetic up to summation order
    assert rel(rounded) < 1e-5 and np.abs(rounded - ref).max() < 1e-3
    # exact products: inside rel-L2 1e-3, outside max-abs 2e-2
    assert rel(exact) < 1e-3
    assert np.abs(exact - ref).max() > 2e-2
