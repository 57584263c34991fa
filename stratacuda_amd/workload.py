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
                 base_seed=BASE_SEED, trace=False, fused=True, prefetch=False):
        """``layers``: a count, or a list of existing DeviceLayer objects
        (layer l of the list is layer l of the stack; not freed here).
        ``fused``: one sm_moe_block call per layer (normalisation and
        residual folded into the stage's kernels) instead of the three
        separate steps; the results are the same bits. ``prefetch``: each
        layer call names the next layer's router matrix (the first layer's
        after the last: the next step's), which a single-launch decode layer
        pulls into L2 (sm_prefetch_router); the same bits."""
        self.b, self.T, self.fused, self.prefetch = backend, tokens, fused, prefetch
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
            if self.prefetch:
                b.prefetch_router(self.layers[(l + 1) % self.L].Wr, self.experts, W)
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


# ---------------------------------------------------------------- packs
# A pack on disk in the reference's strata-pack layout (vendor/strata/tools/
# strata_pack.py:219-263, pack_layer.py:54-115): manifest.json, experts.bin
# holding each layer's blobs back to back (layer l's blob e at the layer's
# offset + e * blob_bytes), and dense.bin holding f32 ("P32") value planes of
# the dense tensors. One extension for this workload, whose shared expert is a
# Q2 blob like the routed ones: manifest.experts.shared lists each layer's
# shared blob in experts.bin (after the routed blobs of every layer).
PACK_FORMAT = "strata-pack"


def blob_offsets(width, ff):
    """Byte offsets of the four planes of a blob (pack_layer.py:54-65)."""
    gu_codes = 0
    d_codes = gu_codes + 2 * ff * width // 4
    gu_scales = d_codes + width * ff // 4
    d_scales = gu_scales + 2 * ff * (width // 64) * 2
    return {"gate_up_codes": gu_codes, "down_codes": d_codes, "gate_up_scales": gu_scales, "down_scales": d_scales}


def write_pack(path, width, ff, experts, topk, layers, name="synthetic MoE pack"):
    """Writes a pack directory. ``layers``: one dict per layer with
    ``arena`` (uint8, experts blobs at `stride`), ``stride``, ``shared``
    (uint8 blob), ``Wr`` (f32 [experts x width]), ``Wsg`` and ``gamma``
    (f32 [width])."""
    import json
    import os
    os.makedirs(path, exist_ok=True)
    bb = blob_bytes(width, ff)
    man = {"format": PACK_FORMAT, "name": name,
           "config": {"width": width, "ff": ff, "experts": experts, "topK": topk, "layers": len(layers)},
           "tensors": {}, "n_experts_per_layer": experts}
    exp_layers, shared, dense_at = [], [], 0
    with open(os.path.join(path, "experts.bin"), "wb") as ef:
        for l, lay in enumerate(layers):
            arena = np.asarray(lay["arena"], np.uint8).reshape(experts, lay["stride"])[:, :bb]
            exp_layers.append({"layer": l, "offset": ef.tell()})
            ef.write(np.ascontiguousarray(arena).tobytes())
        for l, lay in enumerate(layers):
            shared.append({"layer": l, "offset": ef.tell()})
            ef.write(np.asarray(lay["shared"], np.uint8)[:bb].tobytes())
        experts_size = ef.tell()
    with open(os.path.join(path, "dense.bin"), "wb") as df:
        for l, lay in enumerate(layers):
            for tname, key, shape in (("ffn_gate_inp.weight", "Wr", [width, experts]),
                                      ("ffn_gate_inp_shexp.weight", "Wsg", [width]),
                                      ("ffn_norm.weight", "gamma", [width])):
                data = np.asarray(lay[key], np.float32).tobytes()
                man["tensors"]["blk.%d.%s" % (l, tname)] = {
                    "file": "dense.bin", "shape": shape, "form": "P32", "source_type": "F32",
                    "values": {"offset": df.tell(), "bytes": len(data)}}
                df.write(data)
        dense_size = df.tell()
    man["experts"] = {"blob_bytes": bb, "offsets": blob_offsets(width, ff), "layers": exp_layers,
                      "total_bytes": len(layers) * experts * bb, "scales_fp16": True, "source_type": "Q2_0",
                      "form": "S2", "shared": shared}
    man["files"] = {"experts.bin": experts_size, "dense.bin": dense_size}
    with open(os.path.join(path, "manifest.json"), "w") as f:
        json.dump(man, f, indent=1)
    return man


class PackReader:
    """Reads a pack directory with the checks of PackStore (src/model.js:82-103):
    format and expert source type, file sizes against the manifest, plane
    bounds, the blob layout against the geometry."""

    def __init__(self, path):
        import json
        import os
        self.path = path
        self.manifest = man = json.load(open(os.path.join(path, "manifest.json")))
        if man.get("format") != PACK_FORMAT:
            raise ValueError("Expected a Strata canonical pack manifest")
        ex = man.get("experts") or {}
        if ex.get("source_type") != "Q2_0":
            raise ValueError("Canonical expert import currently requires Q2_0; IQ expert packs are not supported")
        c = man["config"]
        self.width, self.ff, self.experts, self.topk, self.layers = (c["width"], c["ff"], c["experts"], c["topK"],
                                                                    c["layers"])
        if self.width % 64 or self.ff % 64:
            raise ValueError("Packed expert dimensions must contain complete groups")
        if ex["blob_bytes"] != blob_bytes(self.width, self.ff) or ex["offsets"] != blob_offsets(self.width, self.ff):
            raise ValueError("expert blob layout does not match the geometry")
        for name, size in man.get("files", {}).items():
            if os.path.getsize(os.path.join(path, name)) != size:
                raise ValueError(name + " size differs from manifest")
        for name, t in man["tensors"].items():
            p = t["values"]
            if p["offset"] < 0 or p["offset"] + p["bytes"] > os.path.getsize(os.path.join(path, t["file"])):
                raise ValueError("Invalid plane " + name + ".values")
            if p["bytes"] != int(np.prod(t["shape"])) * 4:
                raise ValueError("Invalid value plane size: " + name)
        self.blob_bytes = ex["blob_bytes"]

    def dense(self, layer, tname):
        import os
        t = self.manifest["tensors"]["blk.%d.%s" % (layer, tname)]
        with open(os.path.join(self.path, t["file"]), "rb") as f:
            f.seek(t["values"]["offset"])
            data = np.frombuffer(f.read(t["values"]["bytes"]), np.float32).copy()
        if not np.all(np.isfinite(data)):
            raise ValueError("Non-finite model weights")
        return data

    def load_layer(self, backend, layer):
        """The layer resident on the device (a DeviceLayer-shaped object):
        its routed blobs streamed from experts.bin by sm_load_experts."""
        import os
        ex = self.manifest["experts"]
        info = [e for e in ex["layers"] if e["layer"] == layer]
        sh = [e for e in ex.get("shared", []) if e["layer"] == layer]
        if not info or not sh:
            raise ValueError("Layer %d is not in the pack" % layer)
        lay = DeviceLayer.__new__(DeviceLayer)
        lay.b, lay.width, lay.ff, lay.experts = backend, self.width, self.ff, self.experts
        lay.seed, lay.stride = None, blob_stride(self.width, self.ff)
        lay.arena = backend.alloc_bytes(lay.stride * self.experts)
        lay.shared = backend.alloc_bytes(lay.stride)
        f = os.path.join(self.path, "experts.bin")
        scales = ex["offsets"]["gate_up_scales"]
        backend.load_experts(f, info[0]["offset"], self.blob_bytes, self.experts, lay.arena, lay.stride, scales)
        backend.load_experts(f, sh[0]["offset"], self.blob_bytes, 1, lay.shared, lay.stride, scales)
        lay.Wr = backend.alloc(self.dense(layer, "ffn_gate_inp.weight"))
        lay.Wsg = backend.alloc(self.dense(layer, "ffn_gate_inp_shexp.weight"))
        lay.gamma = backend.alloc(self.dense(layer, "ffn_norm.weight"))
        return lay
