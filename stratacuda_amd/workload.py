"""Seeded synthetic MoE-layer workloads (shapes of the StrataCuda MoE path).

Geometry: hidden width 2048, ff 512, 512 experts, top-10 + one shared expert,
Q2 blobs with 64-weight fp16-scale groups (884,736 bytes per expert).

Generation is identical on the device (``Backend.synth_*``) and in the CPU
oracle (``oracle.synth_*``): every tensor is drawn from a counter-based
stream (see ``strata_device.h``) named by (seed, stream):

  router weights W_r [experts x width]   stream 1, sigma 0.02
  shared-expert gate w_sg [width]        stream 2, sigma 0.02
  inter-layer RMSNorm gamma [width]      stream 3, 1 + 0.05 U(-1, 1)
  token inputs X [tokens x width]        stream 4, sigma 1 (decode: RMSNorm'd)
  expert e blob                          stream 16 + e (shared: 16 + experts)

Normals are Irwin-Hall sums of 12 uniforms (mean 0, variance 1, |n| <= 6);
scales are fp16(|0.05 n|); code bytes are uniform (uniform 2-bit codes).
The shared-gate vector's distribution is not fixed by the reference
workload; it is N(0, 0.02^2) here.
"""
import math

import numpy as np

WIDTH, FF, EXPERTS, TOPK = 2048, 512, 512, 10
STREAM_ROUTER, STREAM_SHARED_GATE, STREAM_GAMMA, STREAM_INPUT = 1, 2, 3, 4
STREAM_ZIPF_PERM = 5
STREAM_BLOB0 = 16
ROUTER_SIGMA, GATE_SIGMA, SCALE_SIGMA, GAMMA_AMP = 0.02, 0.02, 0.05, 0.05
BASE_SEED = 20260101


def layer_seed(layer, base=BASE_SEED):
    return base + 7919 * layer


def blob_bytes(width=WIDTH, ff=FF):
    return 2 * ff * width // 4 + width * ff // 4 + 2 * ff * (width // 64) * 2 + width * (ff // 64) * 2


def blob_stride(width=WIDTH, ff=FF):
    """Arena stride: blob size rounded up to 256 bytes."""
    b = blob_bytes(width, ff)
    return (b + 255) // 256 * 256


_M64 = (1 << 64) - 1


def _mix64(z):
    z = (z + 0x9E3779B97F4A7C15) & _M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
    return z ^ (z >> 31)


def rand64(seed, stream, i):
    """rand(seed, stream, i) of the counter-based generator."""
    return _mix64((_mix64((seed + 0x9E3779B97F4A7C15 * (stream + 1)) & _M64) + i) & _M64)


def zipf_bias(experts, seed, s=1.1, lam=1.0):
    """Per-expert router logit bias lam * ln p(pi(e)), p(r) ~ r^-s over ranks
    r = 1..experts, pi a seeded permutation (experts ordered by their draws
    from stream 5). Added to the logits before the router (an elementwise
    add), so about 20 experts take most assignments."""
    draws = np.array([rand64(seed, STREAM_ZIPF_PERM, e) for e in range(experts)], dtype=np.uint64)
    order = np.argsort(draws, kind="stable")  # expert order[r-1] gets rank r
    ranks = np.empty(experts, np.int64)
    ranks[order] = np.arange(1, experts + 1)
    logp = -s * np.log(ranks.astype(np.float64))
    logp -= math.log(np.exp(logp).sum())
    return (lam * logp).astype(np.float32)


class DeviceLayer:
    """One MoE layer's weights resident on the device (all experts in one arena)."""

    def __init__(self, backend, layer=0, width=WIDTH, ff=FF, experts=EXPERTS, base_seed=BASE_SEED):
        self.b = backend
        self.width, self.ff, self.experts = width, ff, experts
        self.seed = layer_seed(layer, base_seed)
        self.stride = blob_stride(width, ff)
        self.arena = backend.alloc_bytes(self.stride * experts)
        self.shared = backend.alloc_bytes(self.stride)
        self.Wr = backend.alloc(experts * width, "f32", zero=False)
        self.Wsg = backend.alloc(width, "f32", zero=False)
        self.gamma = backend.alloc(width, "f32", zero=False)
        backend.synth_blobs(self.arena, experts, width, ff, self.seed, STREAM_BLOB0, SCALE_SIGMA, stride=self.stride)
        backend.synth_blobs(self.shared, 1, width, ff, self.seed, STREAM_BLOB0 + experts, SCALE_SIGMA,
                            stride=self.stride)
        backend.synth_normal(self.Wr, experts * width, self.seed, STREAM_ROUTER, ROUTER_SIGMA)
        backend.synth_normal(self.Wsg, width, self.seed, STREAM_SHARED_GATE, GATE_SIGMA)
        backend.synth_uniform_pm(self.gamma, width, self.seed, STREAM_GAMMA, GAMMA_AMP)

    def free(self):
        for buf in (self.arena, self.shared, self.Wr, self.Wsg, self.gamma):
            self.b.free(buf)


def host_layer(oracle, layer=0, width=WIDTH, ff=FF, experts=EXPERTS, base_seed=BASE_SEED, expert_ids=None):
    """The same layer generated on the host by the oracle. ``expert_ids``
    limits generation to a subset of experts (others stay zero)."""
    seed = layer_seed(layer, base_seed)
    stride = blob_stride(width, ff)
    arena = np.zeros(stride * experts, np.uint8)
    ids = range(experts) if expert_ids is None else sorted(set(int(e) for e in expert_ids))
    for e in ids:
        arena[e * stride:e * stride + blob_bytes(width, ff)] = oracle.synth_blob(width, ff, seed, STREAM_BLOB0 + e,
                                                                                 SCALE_SIGMA)
    shared = np.zeros(stride, np.uint8)
    shared[:blob_bytes(width, ff)] = oracle.synth_blob(width, ff, seed, STREAM_BLOB0 + experts, SCALE_SIGMA)
    return {
        "seed": seed, "stride": stride, "arena": arena, "shared": shared,
        "Wr": oracle.synth_normal(experts * width, seed, STREAM_ROUTER, ROUTER_SIGMA),
        "Wsg": oracle.synth_normal(width, seed, STREAM_SHARED_GATE, GATE_SIGMA),
        "gamma": oracle.synth_uniform_pm(width, seed, STREAM_GAMMA, GAMMA_AMP),
    }


class DeviceStack:
    """The config-5 stack on the device: ``layers`` MoE layers, each step
    h_{l+1} = h_l + MoE_l(RMSNorm(h_l; gamma_l)) for ``tokens`` tokens
    (strata_norm mode 0, eps 1e-6; the layer; strata_elementwise mode 5).
    ``trace`` keeps every layer's input and routing for checking."""

    def __init__(self, backend, layers=48, tokens=1, width=WIDTH, ff=FF, experts=EXPERTS, topk=TOPK,
                 base_seed=BASE_SEED, trace=False, fused=True):
        """``layers``: a count, or a list of existing DeviceLayer objects
        (layer l of the list is layer l of the stack; not freed here).
        ``fused``: one sm_moe_block call per layer (normalisation and
        residual folded into the stage's kernels) instead of the three
        separate steps; the results are the same bits."""
        self.b, self.T, self.fused = backend, tokens, fused
        self.width, self.ff, self.experts, self.topk = width, ff, experts, topk
        self.own_layers = not isinstance(layers, list)
        self.layers = ([DeviceLayer(backend, l, width, ff, experts, base_seed) for l in range(layers)]
                       if self.own_layers else layers)
        self.L = layers = len(self.layers)
        n = tokens * width
        self.H = [backend.alloc(n, zero=False) for _ in range(layers + 1 if trace else 2)]
        self.Xn, self.Y = backend.alloc(n, zero=False), backend.alloc(n, zero=False)
        self.ids = [backend.alloc(tokens * topk, "i32") for _ in range(layers if trace else 1)]
        self.w = [backend.alloc(tokens * topk) for _ in range(layers if trace else 1)]
        self.ws = backend.alloc_bytes(backend.moe_block_workspace_bytes(tokens, width, ff, experts, topk))
        self.trace = trace

    def input(self, seed):
        """Seeded N(0, 1) hidden states for the step's tokens, into H[0]."""
        self.b.synth_normal(self.H[0], self.T * self.width, seed, STREAM_INPUT, 1.0)
        return self.H[0]

    def step(self):
        """Runs every layer once; the result is in self.output()."""
        b, W, T = self.b, self.width, self.T
        for l, lay in enumerate(self.layers):
            h_in = self.H[l if self.trace else l % 2]
            h_out = self.H[l + 1 if self.trace else (l + 1) % 2]
            ids, w = self.ids[l if self.trace else 0], self.w[l if self.trace else 0]
            if self.fused:
                b.moe_block(h_in, T, lay.gamma, 1e-6, lay.Wr, lay.arena, lay.stride, lay.shared, lay.Wsg, W, self.ff,
                            self.experts, self.topk, h_out, ids, w, self.ws)
                continue
            b.run("strata_norm", {"X": h_in, "W": lay.gamma, "Y": self.Xn, "cols": W, "rows": T, "weightRows": 1,
                                  "mode": 0, "epsilon": 1e-6, "scale": 1.0}, [T, 1, 1])
            b.moe_layer(self.Xn, T, lay.Wr, lay.arena, lay.stride, lay.shared, lay.Wsg, W, self.ff, self.experts,
                        self.topk, self.Y, ids, w, self.ws)
            b.run("strata_elementwise", {"A": h_in, "B": self.Y, "Y": h_out, "n": T * W, "mode": 5, "scale": 1.0},
                  [(T * W + 63) // 64, 1, 1])

    def output(self):
        return self.H[self.L if self.trace else self.L % 2]

    def free(self):
        if self.own_layers:
            for lay in self.layers:
                lay.free()
        for buf in self.H + self.ids + self.w + [self.Xn, self.Y, self.ws]:
            self.b.free(buf)
