"""Packed INT4 MLP weight bundles on disk: qweights.bin / scales.bin / metadata.json.

The on-disk format of LeanStream's Ministral packer (examples/ministral/pack/pack_mistral.py:7-48,
reader examples/ministral/python/storage.py:10-66), which is also the layout the MI355X
kernels read from HBM, so a bundle is loaded with two contiguous copies:

* qweights.bin: physical neurons in bundles of `bundle_size`; neuron n's record is
  3 * H / 2 bytes -- its gate row, up row and down column (W_down[:, n]) -- each H signed
  INT4 values in two's complement, -7..7, two per byte, first value in the low nibble.
  A bundle is one LeanStream group (Group2: bundle_size 2, 3 H bytes per group).
* scales.bin: little-endian fp16 [padded_neurons][3][H / 128], one scale per 128 values of
  a row (scale = max |w| / 7 over the block, at least the smallest positive fp16).
* metadata.json: shape, convention strings, bundle geometry, the logical -> physical neuron
  mapping and the quantization error of the packer.

Padded neurons (I rounded up to a whole bundle) have zero weights. Group2 scales viewed per
group are [physical_group, 2, 3, H / 128] (leanstream/integrations/torch/contracts.py:24-47).
"""
import json
from pathlib import Path

import numpy as np

FORMAT = dict(version=0, quant_group_size=128, qvalue_convention="signed_twos_complement_low_nibble_first_-7_to_7",
              vector_order=["gate", "up", "down"], mapping_version=1, scale_dtype="little_endian_float16")
SMALLEST_F16 = np.float16(np.nextafter(np.float16(0), np.float16(1)))


# ------------------------------------------------------------------------- the INT4 format
def quantize_rows(rows, block=128):
    """fp16 rows [..., L] -> (packed uint8 [..., L / 2], fp16 scales [..., L / block]).

    Per block of `block` values: s = fp16(max |w| / 7), at least the smallest positive fp16;
    q = clip(round_half_even(w / s), -7, 7) with the division in fp32; q as a 4-bit two's
    complement nibble, value 2i in the low nibble of byte i."""
    w = np.asarray(rows, dtype=np.float32)
    if w.shape[-1] % block or block % 2:
        raise ValueError("row length must be a multiple of an even block")
    if not np.isfinite(w).all():
        raise ValueError("non-finite weights")
    blocks = w.reshape(*w.shape[:-1], w.shape[-1] // block, block)
    s = (np.abs(blocks).max(axis=-1) / np.float32(7)).astype(np.float16)
    s = np.maximum(s, SMALLEST_F16)
    if not np.isfinite(s).all():
        raise ValueError("fp16 scale overflow")
    q = np.clip(np.rint(blocks / s[..., None].astype(np.float32)), -7, 7).astype(np.int8)
    nib = (q.reshape(w.shape).view(np.uint8) & np.uint8(0xF))
    return (nib[..., 0::2] | (nib[..., 1::2] << np.uint8(4))).astype(np.uint8), s


def unpack_nibbles(packed):
    """uint8 [..., L / 2] -> int8 [..., L] (low nibble first, two's complement)."""
    p = np.asarray(packed, dtype=np.uint8)
    q = np.empty((*p.shape[:-1], 2 * p.shape[-1]), dtype=np.int8)
    q[..., 0::2] = (p & 0xF).astype(np.int8)
    q[..., 1::2] = (p >> 4).astype(np.int8)
    q[q >= 8] -= 16
    return q


def dequantize_rows(packed, scales, block=128):
    """fp16(q * s) per value: the exact weight the kernels multiply."""
    q = unpack_nibbles(packed).astype(np.float32)
    s = np.asarray(scales, dtype=np.float16).astype(np.float32)
    b = q.reshape(*q.shape[:-1], q.shape[-1] // block, block) * s[..., None]
    return b.reshape(q.shape).astype(np.float16)


# ------------------------------------------------------------------------- writing
def write_bundle(path, gate, up, down, bundle_size=2, physical_to_logical=None):
    """Quantize fp16 gate/up [I, H] and down [H, I] into a bundle directory (which must not
    exist). physical_to_logical: physical neuron order (a permutation of range(I)); the
    identity when None. Returns the metadata."""
    gate, up, down = (np.asarray(v, dtype=np.float16) for v in (gate, up, down))
    i, h = gate.shape
    if up.shape != (i, h) or down.shape != (h, i):
        raise ValueError("gate/up must be [I, H] and down [H, I]")
    order = np.arange(i) if physical_to_logical is None else np.asarray(physical_to_logical, dtype=np.int64)
    if bundle_size < 1 or h % 128 or not np.array_equal(np.sort(order), np.arange(i)):
        raise ValueError("bad bundle size, width or mapping")
    padded = -(-i // bundle_size) * bundle_size
    packed = np.zeros((padded, 3, h // 2), dtype=np.uint8)
    scales = np.full((padded, 3, h // 128), SMALLEST_F16, dtype=np.float16)
    rows = np.stack((gate[order], up[order], down[:, order].T), axis=1)   # [I, 3, H] physical order
    packed[:i], scales[:i] = quantize_rows(rows)
    err = np.abs(dequantize_rows(packed[:i], scales[:i]).astype(np.float32) - rows.astype(np.float32))
    return _write(path, packed, scales, h, i, bundle_size, np.argsort(order),
                  mean_absolute_error=float(err.mean()) if err.size else 0.0,
                  max_absolute_error=float(err.max(initial=0.0)))


def write_packed_bundle(path, packed, scales, h, i, bundle_size=2, logical_to_physical=None):
    """A bundle from already packed records [padded, 3, H / 2] and scales [padded, 3, H / 128]."""
    padded = -(-i // bundle_size) * bundle_size
    packed = np.asarray(packed, dtype=np.uint8).reshape(padded, 3, h // 2)
    scales = np.asarray(scales, dtype=np.float16).reshape(padded, 3, h // 128)
    mapping = np.arange(i) if logical_to_physical is None else np.asarray(logical_to_physical, dtype=np.int64)
    return _write(path, packed, scales, h, i, bundle_size, mapping, mean_absolute_error=0.0, max_absolute_error=0.0)


def _write(path, packed, scales, h, i, bundle_size, logical_to_physical, **errors):
    path = Path(path)
    path.mkdir(parents=True, exist_ok=False)
    padded = packed.shape[0]
    (path / "qweights.bin").write_bytes(np.ascontiguousarray(packed).tobytes())
    np.ascontiguousarray(scales).astype("<f2").tofile(path / "scales.bin")
    meta = dict(FORMAT, H=int(h), I=int(i), bundle_size=int(bundle_size), bytes_per_neuron=3 * h // 2,
                bytes_per_bundle=bundle_size * 3 * h // 2, logical_to_physical=[int(v) for v in logical_to_physical],
                padded_neurons=int(padded), **errors)
    (path / "metadata.json").write_text(json.dumps(meta, indent=1) + "\n")
    return meta


# ------------------------------------------------------------------------- reading
class Bundle:
    """A validated bundle (the checks of storage.py:12-35). qweights is memory-mapped."""

    def __init__(self, path):
        self.path = Path(path)
        m = self.meta = json.loads((self.path / "metadata.json").read_text())
        for key, value in FORMAT.items():
            if m.get(key) != value:
                raise ValueError(f"unsupported format: {key} = {m.get(key)!r}")
        h, i, b = m["H"], m["I"], m["bundle_size"]
        if (h % 128 or b < 1 or m["bytes_per_neuron"] != 3 * h // 2 or m["bytes_per_bundle"] != b * 3 * h // 2
                or m["padded_neurons"] != -(-i // b) * b):
            raise ValueError("inconsistent format metadata")
        self.mapping = np.asarray(m["logical_to_physical"], dtype=np.int64)
        if not np.array_equal(np.sort(self.mapping), np.arange(i)):
            raise ValueError("logical_to_physical is not a permutation")
        self.width, self.neurons, self.bundle_size = h, i, b
        self.padded = m["padded_neurons"]
        self.groups = self.padded // b
        self.group_bytes = m["bytes_per_bundle"]
        qpath = self.path / "qweights.bin"
        if qpath.stat().st_size != self.padded * m["bytes_per_neuron"]:
            raise ValueError("qweights.bin has the wrong size")
        scales = np.fromfile(self.path / "scales.bin", dtype="<f2")
        if scales.size != self.padded * 3 * (h // 128):
            raise ValueError("scales.bin has the wrong size")
        self.scales = scales.reshape(self.padded, 3, h // 128)
        if not np.isfinite(self.scales).all() or np.any(self.scales <= 0):
            raise ValueError("scales must be finite and positive")
        self.qweights = np.memmap(qpath, dtype=np.uint8, mode="r", shape=(self.padded, 3, h // 2))

    def group_scales(self):
        """Per-group view [physical_group, bundle_size, 3, H / 128] (Group2 WeightSpec scales)."""
        return self.scales.reshape(self.groups, self.bundle_size, 3, self.width // 128)

    def group_layout(self):
        """GroupLayout records (logical = physical = bundle index, file offset, bytes) for
        HostStagingIO: the bundle file is the host store."""
        rec = np.zeros(self.groups, dtype=[("logical", "<u4"), ("physical", "<u4"), ("offset", "<u8"),
                                           ("bytes", "<u4"), ("reserved", "<u4")])
        rec["logical"] = rec["physical"] = np.arange(self.groups)
        rec["offset"] = np.arange(self.groups, dtype=np.uint64) * np.uint64(self.group_bytes)
        rec["bytes"] = self.group_bytes
        return rec

    def group_of_neuron(self, logical_neuron):
        return self.mapping[np.asarray(logical_neuron)] // self.bundle_size

    def to_device(self, device="cuda"):
        """(cache uint8 [groups * group_bytes], scales fp16 [padded * 3 * H / 128]) on the
        device, in the kernels' layout (one contiguous copy each)."""
        import torch

        cache = torch.from_numpy(np.asarray(self.qweights).reshape(-1)).to(device)
        scales = torch.from_numpy(self.scales.reshape(-1).copy()).to(device)
        return cache, scales

    def dense(self):
        """Dequantized fp16 (gate [I, H], up [I, H], down [H, I]) in logical neuron order."""
        rows = dequantize_rows(np.asarray(self.qweights)[self.mapping], self.scales[self.mapping])
        return rows[:, 0], rows[:, 1], rows[:, 2].T.copy()
