"""The 48-layer stack run free on both sides: the GPU's own trajectory
against the oracle's own f32 trajectory (the reference's per-run route
comparison, reports/model-validation.md:28): the 128 configured decode steps
at batch 1 (the single-launch decode layer) and 4 steps at batch 32 (the
grouped-GEMM path). Layer 0 sees identical inputs, so its routing must be equal; deeper
layers see inputs that differ by the expert products' rounding (within
1e-4 + 1e-3|e| per layer), so a route may flip where two experts'
probabilities are nearly tied. The test reports, per step, the first layer
whose route departs and prints the summary; it requires equal routes at
layer 0 and the layer outputs of both trajectories to stay finite."""
import json
import os

import numpy as np
import pytest

from stratacuda_amd import workload as wl

pytestmark = pytest.mark.gpu

LAYERS = 48


@pytest.fixture(scope="module")
def layers(backend):
    made = [wl.DeviceLayer(backend, l) for l in range(LAYERS)]
    yield made
    for lay in made:
        lay.free()


@pytest.mark.parametrize("tokens,steps", [(1, 128), (32, 4)])
def test_free_running_route_divergence(backend, oracle, layers, tokens, steps):
    W, F, E, K = wl.WIDTH, wl.FF, wl.EXPERTS, wl.TOPK
    st = wl.DeviceStack(backend, layers=layers, tokens=tokens, trace=True)
    seeds = [wl.BASE_SEED + 7000 + 100 * tokens + s for s in range(steps)]
    try:
        gpu_ids = np.zeros((steps, LAYERS, tokens * K), np.int32)
        for s, seed in enumerate(seeds):
            st.input(seed)
            st.step()
            for l in range(LAYERS):
                gpu_ids[s, l] = backend.read(st.ids[l])
    finally:
        st.free()
    # the oracle's trajectory, layer-major over all steps' tokens at once
    # (every token of every step is independent)
    n = steps * tokens
    h = np.concatenate([oracle.synth_normal(tokens * W, seed, wl.STREAM_INPUT, 1.0) for seed in seeds])
    ora_ids = np.zeros_like(gpu_ids)
    for l in range(LAYERS):
        host = wl.host_layer(oracle, l, expert_ids=[])
        xn = oracle.norm(h, host["gamma"], W, n, 1, 0, 1e-6, 1.0)
        rids, _ = oracle.router(oracle.project(xn, host["Wr"], W, E, n), E, K, n)
        host = wl.host_layer(oracle, l, expert_ids=rids)
        h, ids, _ = oracle.moe_block(h, n, host["gamma"], host["Wr"], host["arena"], host["stride"],
                                     host["shared"], host["Wsg"], W, F, E, K)
        assert np.array_equal(ids, rids)
        ora_ids[:, l] = ids.reshape(steps, tokens * K)
        assert np.all(np.isfinite(h)), l
    # per (step, token, layer): the token's K routed IDs equal
    equal = np.all(gpu_ids.reshape(steps, LAYERS, tokens, K) == ora_ids.reshape(steps, LAYERS, tokens, K), axis=3)
    equal = equal.transpose(0, 2, 1).reshape(n, LAYERS)  # [token of a step, layer]
    first = [int(np.argmin(equal[i])) if not equal[i].all() else None for i in range(n)]
    report = {"batch": tokens, "steps": steps, "layers": LAYERS,
              "routes_equal": int(equal.sum()), "routes_compared": int(equal.size),
              "tokens_equal_at_every_layer": int(sum(f is None for f in first)),
              "first_departure_layer": {str(i): f for i, f in enumerate(first) if f is not None}}
    print("free-running routes:", json.dumps(report))
    out = os.environ.get("STRATA_REPORT_DIR")
    if out:
        os.makedirs(out, exist_ok=True)
        with open(os.path.join(out, "stack_free_routes_batch%d.json" % tokens), "w") as f:
            json.dump(report, f, indent=1)
    assert equal[:, 0].all(), "layer-0 routing differs with identical inputs"
