"""Device-resident sparse INT4 MLP layers for tests and benchmarks.

Weights, scales and activations are generated on the GPU by the library's own
generator kernels (identical to leanstream_amd.synth on the host). A layer can be
replicated into several independent copies (different seeds, disjoint memory) so
that a benchmark rotating over them reads HBM rather than the 256 MB Infinity Cache.
"""
import numpy as np

from . import _native, synth
from .backend import MODE_PROGRESSIVE, NativeBackend, ReadyQueue


def _check(rc, what):
    if rc:
        raise RuntimeError(f"{what} failed: {rc}")


class DeviceLayer:
    def __init__(self, cfg, copies=1, logical=None, with_y32=True, diagnostics=True, queue_capacity=None,
                 offline_table=None, stamps=False, claim_log=False, first_compute=False):
        import torch

        self.torch = torch
        self.cfg = cfg
        self.copies = copies
        lib = _native.library()
        dev = torch.device("cuda")
        G, d, n = cfg.group_size, cfg.width, cfg.groups
        stream = torch.cuda.current_stream().cuda_stream
        self.cache = torch.empty(copies * n * cfg.group_bytes, dtype=torch.uint8, device=dev)
        self.scales = torch.empty(copies * n * cfg.scale_words, dtype=torch.float16, device=dev)
        self.x = torch.empty(cfg.batch * d, dtype=torch.float16, device=dev)
        for c in range(copies):
            _check(lib.ls_synth_bytes(self.cache.data_ptr() + c * n * cfg.group_bytes, n * cfg.group_bytes,
                                      cfg.sub_seed(synth.SEED_W) + c * 0x1000, stream), "synth bytes")
            _check(lib.ls_synth_uniform_f16(self.scales.data_ptr() + 2 * c * n * cfg.scale_words, n * cfg.scale_words,
                                            cfg.sub_seed(synth.SEED_S) + c * 0x1000, cfg.scale_lo, cfg.scale_hi,
                                            stream), "synth scales")
        synth_x = lib.ls_synth_normal_bf16 if cfg.x_dtype == "bf16" else lib.ls_synth_normal_f16
        _check(synth_x(self.x.data_ptr(), cfg.batch * d, cfg.sub_seed(synth.SEED_X), stream), "synth x")
        self.logical = synth.active_groups(cfg) if logical is None else np.asarray(logical, dtype=np.int64)
        k = len(self.logical)
        self.k = k
        rows = []
        for c in range(copies):
            r = synth.descriptors(cfg, self.logical)
            r[:, 1] += c * n   # scale rows of copy c
            r[:, 2] += c * n   # cache slots of copy c
            rows.append(r)
        self.core_rows = np.stack(rows)                     # [copies, k, 5]
        self.core = torch.from_numpy(self.core_rows.reshape(-1).astype(np.int32)).to(dev)
        self.slot_capacity = max(1, k)
        self.y = torch.empty(cfg.batch * d, dtype=torch.float16, device=dev)
        self.y32 = torch.empty(cfg.batch * d, dtype=torch.float32, device=dev) if with_y32 else None
        # h of each destination row and batch row: fp32 bits in the low word, launch
        # sequence tag in the high word ([slot][batch][G])
        self.hidden = torch.zeros(self.slot_capacity * cfg.batch * G, dtype=torch.int64, device=dev)
        self.executions = torch.zeros(self.slot_capacity, dtype=torch.int32, device=dev) if diagnostics else None
        self.queue = ReadyQueue(queue_capacity if queue_capacity else max(1, k))
        self.stamps = torch.zeros(4096 * 32, dtype=torch.int64, device=dev) if stamps else None
        # claim log: 4 words per range a workgroup takes (candidates that consume the queue in
        # ranges), at most one range per queue position
        self.claim_log = (torch.zeros(self.queue.capacity * 4, dtype=torch.int32, device=dev) if claim_log
                          else None)
        # first compute stamp of each destination row (100 MHz device clock)
        self.first_compute = (torch.zeros(self.slot_capacity, dtype=torch.int64, device=dev) if first_compute
                              else None)
        self.backend = NativeBackend(offline_table)
        self.backend.bind(d, G, self.slot_capacity, self.cache, self.scales, physical_groups=copies * n,
                          cache_groups=copies * n, staging=self.cache, staging_groups=copies * n,
                          queue_capacity=self.queue.capacity, hidden=self.hidden, y32=self.y32,
                          executions=self.executions, batch=cfg.batch, stamps=self.stamps,
                          claim_log=self.claim_log, first_compute=self.first_compute)
        torch.cuda.synchronize()

    def core_ptr(self, copy):
        return self.core.data_ptr() + copy * self.k * 20

    def seal_empty_queue(self, epoch):
        self.queue.reset(epoch)
        self.queue.seal(0)

    def run_core(self, copy=0, epoch=1, layer=0, bucket=0, stream=None, mode=MODE_PROGRESSIVE):
        """Enqueue one layer whose active groups are all resident core descriptors."""
        torch = self.torch
        s = stream if stream is not None else torch.cuda.current_stream().cuda_stream
        self.backend.enqueue(layer, bucket, epoch, self.x, self.y, s, self.core_ptr(copy), self.k, self.queue, mode)

    def chain_outputs(self, count):
        """Per-layer output rows of a chain of `count` layers: y (fp16), y32, hidden (fp16)."""
        torch = self.torch
        d = self.cfg.width
        return (torch.empty(count, d, dtype=torch.float16, device="cuda"),
                torch.empty(count, d, dtype=torch.float32, device="cuda"),
                torch.empty(count, d, dtype=torch.float16, device="cuda"))

    def chain_norm_weights(self, count, seed=29, lo=0.05, hi=0.15):
        """Per-layer RMSNorm weights (fp16 U(lo, hi), seeded) for a chain of `count` layers.
        With random layer weights the layer output grows with the square of its input; inputs
        of rms ~0.1 keep each layer's output small next to the residual stream, so the stream
        of 36 layers stays bounded (with weights near 1 it grows past fp16 within six layers
        of the Ministral-8B shape, in the oracle's arithmetic as on the GPU)."""
        torch = self.torch
        rng = np.random.default_rng(seed)
        w = rng.uniform(lo, hi, (count, self.cfg.width)).astype(np.float16)
        return torch.from_numpy(w).cuda()

    def chain_layers(self, order, outputs, x=None, epoch0=1, flags=None, output32=True, norm=None, eps=1e-5,
                     residual=None):
        """ls_hip_chain_layer blocks of a chain whose layer i runs copy order[i] of this layer:
        the first reads x (default self.x) and `residual` (default: x); every later one takes
        the previous hidden state as its residual and as its input, or RMSNorm of it times
        norm[i] (norm: [count, d] fp16 weights). flags: optional (flag address per layer, bell
        address) host-coherent words."""
        y, y32, hidden = outputs
        n = self.cfg.groups
        layers = []
        for i, c in enumerate(order):
            layer = dict(core=self.core_ptr(c), core_count=self.k, cache=self.cache, cache_groups=self.copies * n,
                         scales=self.scales, physical_groups=self.copies * n, output=y[i], hidden=hidden[i],
                         epoch=epoch0 + i, norm_eps=eps)
            if output32:
                layer["output32"] = y32[i]
            if i == 0:
                layer["input"] = self.x if x is None else x
                if residual is not None:
                    layer["residual"] = residual
            elif norm is not None:
                layer["norm_weight"] = norm[i]
            if flags is not None:
                layer["hidden_flag"] = flags[0] + 4 * i
                layer["bell"] = flags[1]
            layers.append(layer)
        return layers

    def copy_rows(self, copy):
        """Host (numpy) cache and scales of one copy, and its descriptors relative to it."""
        n = self.cfg.groups
        cache = self.cache[copy * n * self.cfg.group_bytes:(copy + 1) * n * self.cfg.group_bytes].cpu().numpy()
        scales = self.scales[copy * n * self.cfg.scale_words:(copy + 1) * n * self.cfg.scale_words].cpu().numpy()
        return synth.descriptors(self.cfg, self.logical), cache, scales

    def hidden_h(self):
        """h per destination row and neuron (fp32) from the tagged hidden buffer."""
        words = self.hidden.cpu().numpy().view(np.uint32).reshape(-1, 2)[:, 0]
        h = words.view(np.float32).reshape(self.slot_capacity, self.cfg.batch, self.cfg.group_size)
        return h[:, 0, :] if self.cfg.batch == 1 else h

    def host_copy(self):
        """Host (numpy) copies of copy 0: cache, scales, x."""
        n = self.cfg.groups
        cache = self.cache[: n * self.cfg.group_bytes].cpu().numpy()
        scales = self.scales[: n * self.cfg.scale_words].cpu().numpy()
        return cache, scales, self.x.cpu().numpy()

    def close(self):
        self.torch.cuda.synchronize()
        self.backend.close()
        self.queue.close()
