"""The packed INT4 bundle format (leanstream_amd/weights.py; LeanStream
examples/ministral/pack/pack_mistral.py:7-48, int4_format.py, python/storage.py:10-66) on the CPU:
the nibble and scale convention from first principles, the round-trip error bound, the
reader's validation, and that a bundle's bytes are the layout the kernels and the oracle read
(group = bundle; neuron record gate | up | down column), checked against a dense layer
computed from the dequantized weights."""
import json

import numpy as np
import pytest

import oracle
from leanstream_amd import synth, weights


def test_nibble_and_scale_convention():
    # block max 7 -> scale 1: the values themselves; two's complement, low nibble first
    row = np.zeros(128, dtype=np.float16)
    row[:6] = [1, -1, 7, -7, 0, 3]
    packed, s = weights.quantize_rows(row)
    assert s.shape == (1,) and s[0] == np.float16(1.0)
    assert packed[:3].tolist() == [0xF1, 0x97, 0x30]
    assert np.array_equal(weights.unpack_nibbles(packed)[:6], [1, -1, 7, -7, 0, 3])
    # an all-zero block keeps the smallest positive scale (readers reject scale <= 0)
    _, s0 = weights.quantize_rows(np.zeros(256, dtype=np.float16))
    assert np.all(s0 == weights.SMALLEST_F16) and np.all(s0 > 0)
    # -8 is never produced; rounding is half to even on w / s
    _, s = weights.quantize_rows(np.full(128, 3.5, dtype=np.float16))
    q = weights.unpack_nibbles(weights.quantize_rows(np.r_[np.full(127, 3.5), [1.25]].astype(np.float16))[0])
    assert q.min() >= -7 and q[0] == 7 and q[-1] == np.rint(1.25 / (3.5 / 7))


def test_round_trip_error_is_at_most_half_a_step():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((8, 3, 512)) * rng.uniform(0.01, 3, (8, 3, 1))).astype(np.float16)
    packed, s = weights.quantize_rows(w)
    d = weights.dequantize_rows(packed, s).astype(np.float64)
    step = np.repeat(s.astype(np.float64), 128, axis=-1)
    # |q s - w| <= s / 2, plus the fp16 rounding of q s
    assert np.all(np.abs(d - w.astype(np.float64)) <= step / 2 + np.abs(d) * 2.0 ** -11 + 1e-12)


def _small_layer(i=60, h=256, seed=5):
    rng = np.random.default_rng(seed)
    gate = (rng.standard_normal((i, h)) * 0.05).astype(np.float16)
    up = (rng.standard_normal((i, h)) * 0.05).astype(np.float16)
    down = (rng.standard_normal((h, i)) * 0.05).astype(np.float16)
    return gate, up, down


def test_write_and_read_bundle(tmp_path):
    gate, up, down = _small_layer(i=61)          # not a multiple of the bundle: one padded neuron
    order = synth.permutation(61, 9)
    meta = weights.write_bundle(tmp_path / "l0", gate, up, down, bundle_size=2, physical_to_logical=order)
    b = weights.Bundle(tmp_path / "l0")
    assert (b.width, b.neurons, b.padded, b.groups, b.group_bytes) == (256, 61, 62, 31, 768)
    assert meta["bytes_per_bundle"] == 768 and meta["max_absolute_error"] > 0
    assert np.array_equal(b.mapping, np.argsort(order))
    assert b.group_scales().shape == (31, 2, 3, 2)
    assert np.all(np.asarray(b.qweights)[61] == 0)              # padding
    g2, u2, d2 = b.dense()
    for a, ref in ((g2, gate), (u2, up), (d2, down)):
        assert np.abs(a.astype(np.float32) - ref.astype(np.float32)).max() <= meta["max_absolute_error"] + 1e-6
    rec = b.group_layout()
    assert rec["offset"][5] == 5 * 768 and np.all(rec["bytes"] == 768)
    # a neuron's group is its physical bundle
    assert b.group_of_neuron(int(order[7])) == 3


@pytest.mark.parametrize("change", ["convention", "size", "mapping", "scale"])
def test_reader_rejects_inconsistent_bundles(tmp_path, change):
    gate, up, down = _small_layer(i=8)
    p = tmp_path / "l"
    weights.write_bundle(p, gate, up, down, bundle_size=2)
    meta = json.loads((p / "metadata.json").read_text())
    if change == "convention":
        meta["qvalue_convention"] = "unsigned"
    elif change == "mapping":
        meta["logical_to_physical"][0] = meta["logical_to_physical"][1]
    if change in ("convention", "mapping"):
        (p / "metadata.json").write_text(json.dumps(meta))
    elif change == "size":
        (p / "qweights.bin").write_bytes((p / "qweights.bin").read_bytes()[:-1])
    else:
        s = np.fromfile(p / "scales.bin", dtype="<f2")
        s[3] = 0
        s.tofile(p / "scales.bin")
    with pytest.raises(ValueError):
        weights.Bundle(p)


def _dense_layer(gate, up, down, x, neurons):
    """The layer over `neurons` from dense fp16 weights, rounding to fp16 where the kernels
    do (g, u, silu, h), accumulating in float64."""
    xf = x.astype(np.float64)
    g = (gate[neurons].astype(np.float64) @ xf).astype(np.float16).astype(np.float64)
    u = (up[neurons].astype(np.float64) @ xf).astype(np.float16).astype(np.float64)
    silu = (g / (1 + np.exp(-g))).astype(np.float16).astype(np.float64)
    hh = (silu * u).astype(np.float16).astype(np.float64)
    return down[:, neurons].astype(np.float64) @ hh


def test_bundle_bytes_are_the_kernel_layout(tmp_path):
    """The oracle (the kernels' arithmetic on packed groups) over a bundle's bytes equals the
    layer computed from the bundle's dequantized dense weights."""
    gate, up, down = _small_layer(i=64, h=512, seed=11)
    order = synth.permutation(64, 4)
    weights.write_bundle(tmp_path / "l", gate, up, down, bundle_size=2, physical_to_logical=order)
    b = weights.Bundle(tmp_path / "l")
    g2, u2, d2 = b.dense()
    x = synth.normal_f16(512, 77)
    active = np.array([3, 17, 0, 30, 9, 21])                    # groups = physical bundles
    descs = np.zeros((len(active), 5), dtype=np.uint32)
    descs[:, 0] = descs[:, 1] = descs[:, 2] = active
    descs[:, 3] = np.arange(len(active))
    ref = oracle.layer(descs, len(active), np.asarray(b.qweights).reshape(-1), b.scales.reshape(-1), x, 512, 2)
    neurons = np.concatenate([order[2 * g:2 * g + 2] for g in active])   # logical neurons of the groups
    want = _dense_layer(g2, u2, d2, x, neurons)
    rel = np.linalg.norm(ref["y32"] - want) / np.linalg.norm(want)
    assert rel < 1e-5, rel
    # a transposed down projection or swapped gate/up is caught
    wrong = _dense_layer(u2, g2, d2, x, neurons)
    assert np.linalg.norm(ref["y32"] - wrong) / np.linalg.norm(wrong) > 1e-2
