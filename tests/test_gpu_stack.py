"""The 48-layer stack of the MoE path (h <- h + MoE_l(RMSNorm(h; gamma_l)))
on the GPU, teacher-forced against the CPU oracle: every layer's routing is
recomputed by the oracle from the GPU's own input to that layer, so routed
IDs and their order must match bit for bit at every layer of all 128
configured steps, at batch 1 and at batch 32, and the routing weights bit for
bit (both batches are below the certified router's 512 tokens), and every
layer's output within
|a - e| <= 1e-4 + 1e-3 |e| (the f32 trajectory itself is not bit-exact: the
fused expert products only meet the tolerance;
tests/test_gpu_stack_free.py follows the two trajectories apart)."""
import numpy as np
import pytest

from conftest import tol_ok, weights_ok
from stratacuda_amd import workload as wl

pytestmark = pytest.mark.gpu

LAYERS = 48


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


STEPS = 128  # the configured decode length


@pytest.fixture(scope="module")
def stack_layers(backend):
    layers = [wl.DeviceLayer(backend, l) for l in range(LAYERS)]
    yield layers
    for lay in layers:
        lay.free()


@pytest.fixture(scope="module")
def router_weights(backend, stack_layers):
    """Host copies of every layer's router matrix and RMSNorm gamma."""
    return [(backend.read(lay.Wr), backend.read(lay.gamma)) for lay in stack_layers]


def oracle_routing(oracle, h, tokens, Wr, gamma):
    """strata_norm mode 0, the router projection and strata_router, in the
    reference's order, for `tokens` rows of the layer input h."""
    xn = oracle.norm(h, gamma, wl.WIDTH, tokens, 1, 0, 1e-6, 1.0)
    logits = oracle.project(xn, Wr, wl.WIDTH, wl.EXPERTS, tokens)
    return oracle.router(logits, wl.EXPERTS, wl.TOPK, tokens)


def teacher_forced_routing(backend, oracle, st, router_weights, tokens):
    """Every layer's routed IDs and weights against the oracle's routing of
    the GPU's own input to that layer; returns the number of layers checked."""
    for l in range(LAYERS):
        Wr, gamma = router_weights[l]
        rids, rw = oracle_routing(oracle, backend.read(st.H[l]), tokens, Wr, gamma)
        assert np.array_equal(backend.read(st.ids[l]), rids), "layer %d routing differs" % l
        assert weights_ok(tokens, backend.read(st.w[l]), rw), "layer %d routing weights differ" % l
    return LAYERS


def check_layer(backend, oracle, st, l, rows):
    W, K = wl.WIDTH, wl.TOPK
    h_in = backend.read(st.H[l]).reshape(st.T, W)
    h_out = backend.read(st.H[l + 1]).reshape(st.T, W)
    ids = backend.read(st.ids[l]).reshape(st.T, K)
    w = backend.read(st.w[l]).reshape(st.T, K)
    sub = ids[rows].reshape(-1)
    host = wl.host_layer(oracle, l, expert_ids=sub)
    out, eids, ew = oracle.moe_block(h_in[rows].reshape(-1), len(rows), host["gamma"], host["Wr"], host["arena"],
                                     host["stride"], host["shared"], host["Wsg"], W, wl.FF, wl.EXPERTS, K)
    assert np.array_equal(eids, sub), "layer %d routing differs" % l
    assert weights_ok(st.T, w[rows].reshape(-1), ew), "layer %d routing weights differ" % l
    got = h_out[rows].reshape(-1)
    assert tol_ok(got, out), "layer %d output: max abs err %g" % (l, np.abs(got - out).max())


def test_stack_decode_batch1_every_layer(backend, oracle, stack_layers):
    st = wl.DeviceStack(backend, layers=stack_layers, tokens=1, trace=True)
    try:
        for step in range(2):
            st.input(wl.BASE_SEED + 1000 + step)
            st.step()
            assert np.all(np.isfinite(backend.read(st.output())))
            for l in range(LAYERS):
                check_layer(backend, oracle, st, l, [0])
    finally:
        st.free()


def test_stack_decode_batch1_all_steps_routing(backend, oracle, stack_layers, router_weights):
    # The configured 128 decode steps at batch 1, each from its own seeded
    # N(0, 1) input: every layer's routing, teacher-forced, bit-exact.
    st = wl.DeviceStack(backend, layers=stack_layers, tokens=1, trace=True)
    try:
        checked = 0
        for step in range(STEPS):
            st.input(wl.BASE_SEED + 5000 + step)
            st.step()
            assert np.all(np.isfinite(backend.read(st.output()))), step
            checked += teacher_forced_routing(backend, oracle, st, router_weights, 1)
        assert checked == STEPS * LAYERS
    finally:
        st.free()


@pytest.mark.parametrize("half", [0, 1])
def test_stack_batch32_all_steps_routing(backend, oracle, stack_layers, router_weights, half):
    # All 128 batch-32 steps (in two halves, each its own test): all 32
    # tokens' routing at every layer, teacher-forced, IDs bit-exact.
    st = wl.DeviceStack(backend, layers=stack_layers, tokens=32, trace=True)
    try:
        checked = 0
        for step in range(half * STEPS // 2, (half + 1) * STEPS // 2):
            st.input(wl.BASE_SEED + 9000 + step)
            st.step()
            checked += teacher_forced_routing(backend, oracle, st, router_weights, 32)
        assert checked == STEPS // 2 * LAYERS
    finally:
        st.free()


def test_stack_batch32(backend, oracle, stack_layers):
    st = wl.DeviceStack(backend, layers=stack_layers, tokens=32, trace=True)
    try:
        st.input(wl.BASE_SEED + 2000)
        st.step()
        assert np.all(np.isfinite(backend.read(st.output())))
        # routing of all 32 tokens at every layer, bit-exact, from the GPU's layer inputs
        for l in range(LAYERS):
            h_in = backend.read(st.H[l])
            lay = stack_layers[l]
            xn = oracle.norm(h_in, backend.read(lay.gamma), wl.WIDTH, 32, 1, 0, 1e-6, 1.0)
            logits = oracle.project(xn, backend.read(lay.Wr), wl.WIDTH, wl.EXPERTS, 32)
            rids, rw = oracle.router(logits, wl.EXPERTS, wl.TOPK, 32)
            assert np.array_equal(backend.read(st.ids[l]), rids), "layer %d routing differs" % l
            assert weights_ok(32, backend.read(st.w[l]), rw), "layer %d routing weights differ" % l
        # every token's output at the first, middle and last layers
        for l in (0, LAYERS // 2, LAYERS - 1):
            check_layer(backend, oracle, st, l, list(range(32)))
    finally:
        st.free()


@pytest.mark.parametrize("tokens", [1, 4, 8, 32, 100, 512])
def test_block_entry_matches_separate_steps(backend, stack_layers, tokens):
    """sm_moe_block (normalisation and residual folded into the stage) gives
    the same bits as strata_norm, sm_moe_layer and strata_elementwise run
    one after the other, over four layers, also when writing in place."""
    fused = wl.DeviceStack(backend, layers=stack_layers[:4], tokens=tokens, trace=True, fused=True)
    split = wl.DeviceStack(backend, layers=stack_layers[:4], tokens=tokens, trace=True, fused=False)
    try:
        for st in (fused, split):
            st.input(wl.BASE_SEED + 77 + tokens)
            st.step()
        for l in range(1, 5):
            assert same_bits(backend.read(fused.H[l]), backend.read(split.H[l])), "layer %d" % (l - 1)
            assert np.array_equal(backend.read(fused.ids[l - 1]), backend.read(split.ids[l - 1]))
        # in place: H <- H + MoE(RMSNorm(H))
        lay = stack_layers[0]
        W = wl.WIDTH
        backend.copy(split.H[0], fused.H[1], tokens * W)
        backend.moe_block(fused.H[1], tokens, lay.gamma, 1e-6, lay.Wr, lay.arena, lay.stride, lay.shared, lay.Wsg,
                          W, wl.FF, wl.EXPERTS, wl.TOPK, fused.H[1], fused.ids[0], fused.w[0], fused.ws)
        assert same_bits(backend.read(fused.H[1]), backend.read(split.H[1]))
    finally:
        fused.free()
        split.free()
