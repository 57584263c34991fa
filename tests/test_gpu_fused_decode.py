"""The single-launch decode layer (one token, hidden 2048 / ff 512, and the
real model's hidden 2560 / ff 640) against
the three-kernel decode path and the CPU oracle: the same bits as the three
kernels (both compute every product and sum in the same order), routing
bit-exact with the oracle, and no wait ever giving up (fusedDecodeFault 0)
over many launches in a row, across layers and replayed from a graph: each
launch takes the number after the go word the previous one left, so no
counter is reset between launches. The give-up path is forced from the host
(a low poll limit and a collector waiting for a flag no block writes, so
every kernel still ends normally): NaN outputs, SM_E_FAULT from sync and
read, the fault sticky until sm_fused_reset, bit-exact results after it."""
import numpy as np
import pytest

import stratacuda_amd as sm
from conftest import tol_ok
from stratacuda_amd import workload as wl

pytestmark = pytest.mark.gpu

ALL = 0xffffffff
THREE_KERNELS = ALL & ~(1 << 8)  # stage 8 off: the decode stages as three launches


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def two_layers(backend):
    ls = [wl.DeviceLayer(backend, layer=l) for l in (5, 6)]
    yield ls
    for l in ls:
        l.free()


def run_layer(b, lay, X, Y, ids, w, ws, mask, block=False, Hout=None, E=wl.EXPERTS, K=wl.TOPK, bias=None,
              W=wl.WIDTH, F=wl.FF):
    b.stage_select(mask)
    try:
        if block:
            b.moe_block(X, 1, lay.gamma, 1e-6, lay.Wr, lay.arena, lay.stride, lay.shared, lay.Wsg, W, F, E, K,
                        Hout, ids, w, ws, bias=bias)
        else:
            b.moe_layer(X, 1, lay.Wr, lay.arena, lay.stride, lay.shared, lay.Wsg, W, F, E, K, Y, ids, w, ws,
                        bias=bias)
    finally:
        b.stage_select()


@pytest.mark.parametrize("block", [False, True])
@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_fused_matches_three_kernels(backend, two_layers, block, seed):
    b = backend
    W, F, E, K = wl.WIDTH, wl.FF, wl.EXPERTS, wl.TOPK
    lay = two_layers[seed % 2]
    X = b.alloc(W, zero=False)
    b.synth_normal(X, W, 600 + seed, wl.STREAM_INPUT, 1.0)
    ws = b.alloc_bytes(b.moe_block_workspace_bytes(1, W, F, E, K))
    outs = []
    for mask in (ALL, THREE_KERNELS):
        Y, ids, w = b.alloc(W), b.alloc(K, "i32"), b.alloc(K)
        run_layer(b, lay, X, Y, ids, w, ws, mask, block=block, Hout=Y)
        outs.append((b.read(Y), b.read(ids), b.read(w)))
    (y0, i0, w0), (y1, i1, w1) = outs
    assert np.array_equal(i0, i1)
    assert np.array_equal(bits(w0), bits(w1))
    assert np.all(np.isfinite(y0))
    assert np.array_equal(bits(y0), bits(y1)), float(np.abs(y0 - y1).max())
    assert b.info()["fusedDecodeFault"] == 0


def test_fused_block_in_place(backend, two_layers):
    # Hout == H: every block reads all of H before any block writes its rows.
    b = backend
    W, F, E, K = wl.WIDTH, wl.FF, wl.EXPERTS, wl.TOPK
    lay = two_layers[0]
    H1, H2 = b.alloc(W, zero=False), b.alloc(W, zero=False)
    b.synth_normal(H1, W, 77, wl.STREAM_INPUT, 1.0)
    b.copy(H1, H2)
    Hout = b.alloc(W)
    ws = b.alloc_bytes(b.moe_block_workspace_bytes(1, W, F, E, K))
    ids, w = b.alloc(K, "i32"), b.alloc(K)
    run_layer(b, lay, H1, None, ids, w, ws, THREE_KERNELS, block=True, Hout=Hout)
    run_layer(b, lay, H2, None, ids, w, ws, ALL, block=True, Hout=H2)
    assert np.array_equal(bits(b.read(H2)), bits(b.read(Hout)))


def test_many_launches_in_a_row(backend, two_layers):
    # 96 launches back to back (layers alternating, inputs changing), then the
    # same sequence replayed from a graph three times: each launch's result
    # equals the three-kernel result for its input; no wait ever gave up.
    b = backend
    W, F, E, K = wl.WIDTH, wl.FF, wl.EXPERTS, wl.TOPK
    n = 96
    X = b.alloc(n * W, zero=False)
    b.synth_normal(X, n * W, 991, wl.STREAM_INPUT, 1.0)
    xs = [b.alloc(W, zero=False) for _ in range(n)]
    for i in range(n):
        b.copy(X, xs[i], W, i * W, 0)
    ws = b.alloc_bytes(b.moe_workspace_bytes(1, W, F, E, K))
    ref = []
    for i in range(n):
        Y, ids, w = b.alloc(W), b.alloc(K, "i32"), b.alloc(K)
        run_layer(b, two_layers[i % 2], xs[i], Y, ids, w, ws, THREE_KERNELS)
        ref.append((Y, ids, w))
    outs = [(b.alloc(W), b.alloc(K, "i32"), b.alloc(K)) for _ in range(n)]

    def sequence():
        for i in range(n):
            run_layer(b, two_layers[i % 2], xs[i], *outs[i], ws, ALL)

    def check(tag):
        for i in range(n):
            assert np.array_equal(bits(b.read(outs[i][0])), bits(b.read(ref[i][0]))), (tag, i)
            assert np.array_equal(b.read(outs[i][1]), b.read(ref[i][1])), (tag, i)
        for o in outs:
            b.zero(o[0])

    sequence()
    check("eager")
    b.graph_begin()
    sequence()
    gid = b.graph_end()
    for rep in range(3):
        b.graph_launch(gid)
        b.sync()
        check("replay %d" % rep)
    b.graph_free(gid)
    assert b.info()["fusedDecodeFault"] == 0


@pytest.mark.parametrize("experts,topk", [(512, 4), (300, 10), (130, 7), (512, 1)])
def test_fused_other_routing_shapes(backend, oracle, experts, topk):
    # Fewer experts (router rows past `experts` idle) and smaller top-k
    # (waves past topk x 512 hidden rows idle), against the oracle.
    b = backend
    W, F = wl.WIDTH, wl.FF
    lay = wl.DeviceLayer(b, layer=9, experts=experts)
    X = b.alloc(W, zero=False)
    b.synth_normal(X, W, 4000 + experts + topk, wl.STREAM_INPUT, 1.0)
    ws = b.alloc_bytes(b.moe_workspace_bytes(1, W, F, experts, topk))
    Y, ids, w = b.alloc(W), b.alloc(topk, "i32"), b.alloc(topk)
    Y3, ids3, w3 = b.alloc(W), b.alloc(topk, "i32"), b.alloc(topk)
    run_layer(b, lay, X, Y, ids, w, ws, ALL, E=experts, K=topk)
    run_layer(b, lay, X, Y3, ids3, w3, ws, THREE_KERNELS, E=experts, K=topk)
    got_ids = b.read(ids)
    host = wl.host_layer(oracle, 9, experts=experts, expert_ids=list(got_ids))
    eY, eids, ew = oracle.moe_layer(b.read(X), 1, host["Wr"], host["arena"], host["stride"], host["shared"],
                                    host["Wsg"], W, F, experts, topk)
    lay.free()
    assert np.array_equal(got_ids, eids)
    assert np.array_equal(bits(b.read(w)), bits(ew))
    got = b.read(Y)
    assert tol_ok(got, eY), float(np.abs(got - eY).max())
    assert np.array_equal(bits(got), bits(b.read(Y3)))
    assert b.info()["fusedDecodeFault"] == 0


def test_fused_stage_timing(backend, two_layers):
    # With stage timing on, the single launch is reported as stage 8.
    b = backend
    W, F, E, K = wl.WIDTH, wl.FF, wl.EXPERTS, wl.TOPK
    X = b.alloc(W, zero=False)
    b.synth_normal(X, W, 5, wl.STREAM_INPUT, 1.0)
    ws = b.alloc_bytes(b.moe_workspace_bytes(1, W, F, E, K))
    Y, ids, w = b.alloc(W), b.alloc(K, "i32"), b.alloc(K)
    b.stage_timing(True)
    for _ in range(4):
        run_layer(b, two_layers[0], X, Y, ids, w, ws, ALL)
    rep = b.stage_report()
    b.stage_timing(False)
    assert rep["decode_fused"][1] == 4
    assert rep["decode_route"][1] == 0


def test_fused_give_up_reported_and_reset(backend, two_layers):
    b = backend
    W, F, E, K = wl.WIDTH, wl.FF, wl.EXPERTS, wl.TOPK
    assert b.info()["fusedDecode"] is True  # 256 CUs on an MI355X, one block each
    lay = two_layers[0]
    X = b.alloc(W, zero=False)
    b.synth_normal(X, W, 31, wl.STREAM_INPUT, 1.0)
    ws = b.alloc_bytes(b.moe_workspace_bytes(1, W, F, E, K))
    ids, w = b.alloc(K, "i32"), b.alloc(K)
    Y0, Y1, Y2, Y3 = (b.alloc(W) for _ in range(4))
    run_layer(b, lay, X, Y0, ids, w, ws, ALL)
    y0 = b.read(Y0)
    assert np.all(np.isfinite(y0))
    try:
        b.fused_test_hooks(spin_limit=64, withhold=True)
        print("fused give-up: withheld launch", flush=True)
        run_layer(b, lay, X, Y1, ids, w, ws, ALL)
        with pytest.raises(sm.StrataError) as err:
            b.idle()
        assert err.value.code == sm.SM_E_FAULT
        with pytest.raises(sm.StrataError) as err:
            b.read(Y1)
        assert err.value.code == sm.SM_E_FAULT
        b.fused_test_hooks()
        # sticky: a launch with every wait satisfied still writes NaN
        run_layer(b, lay, X, Y2, ids, w, ws, ALL)
        with pytest.raises(sm.StrataError):
            b.idle()
        assert b.info()["fusedDecodeFault"] == 1
    finally:
        b.fused_test_hooks()
        b.fused_reset()
    assert b.info()["fusedDecodeFault"] == 0
    assert np.all(np.isnan(b.read(Y1))) and np.all(np.isnan(b.read(Y2)))
    print("fused give-up: launch after reset", flush=True)
    run_layer(b, lay, X, Y3, ids, w, ws, ALL)
    assert np.array_equal(bits(b.read(Y3)), bits(y0))
    # and again, from the three kernels' side: the same bits
    run_layer(b, lay, X, Y1, ids, w, ws, THREE_KERNELS)
    assert np.array_equal(bits(b.read(Y1)), bits(y0))
    assert b.info()["fusedDecodeFault"] == 0


# The real model's geometry (src/model.js:4-6): hidden 2560, expert ff 640.
RW, RF = 2560, 640


@pytest.fixture(scope="module")
def rg_layers(backend):
    ls = [wl.DeviceLayer(backend, layer=l, width=RW, ff=RF, experts=wl.EXPERTS, base_seed=wl.BASE_SEED + 1)
          for l in (2, 3)]
    yield ls
    for l in ls:
        l.free()


def test_fused_2560_enabled(backend):
    assert backend.info()["fusedDecode2560"] is True


@pytest.mark.parametrize("block", [False, True])
@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_fused_2560_matches_three_kernels(backend, rg_layers, block, seed):
    b = backend
    E, K = wl.EXPERTS, wl.TOPK
    lay = rg_layers[seed % 2]
    X = b.alloc(RW, zero=False)
    b.synth_normal(X, RW, 700 + seed, wl.STREAM_INPUT, 1.0)
    ws = b.alloc_bytes(b.moe_block_workspace_bytes(1, RW, RF, E, K))
    outs = []
    for mask in (ALL, THREE_KERNELS):
        Y, ids, w = b.alloc(RW), b.alloc(K, "i32"), b.alloc(K)
        run_layer(b, lay, X, Y, ids, w, ws, mask, block=block, Hout=Y, W=RW, F=RF)
        outs.append((b.read(Y), b.read(ids), b.read(w)))
    (y0, i0, w0), (y1, i1, w1) = outs
    assert np.array_equal(i0, i1)
    assert np.array_equal(bits(w0), bits(w1))
    assert np.all(np.isfinite(y0))
    assert np.array_equal(bits(y0), bits(y1)), float(np.abs(y0 - y1).max())
    assert b.info()["fusedDecodeFault"] == 0


def test_fused_2560_many_launches(backend, rg_layers):
    # 48 launches back to back and replayed from a graph twice, each equal to
    # the three-kernel result for its input.
    b = backend
    E, K = wl.EXPERTS, wl.TOPK
    n = 48
    xs = []
    for i in range(n):
        x = b.alloc(RW, zero=False)
        b.synth_normal(x, RW, 1300 + i, wl.STREAM_INPUT, 1.0)
        xs.append(x)
    ws = b.alloc_bytes(b.moe_workspace_bytes(1, RW, RF, E, K))
    ref = []
    for i in range(n):
        Y, ids, w = b.alloc(RW), b.alloc(K, "i32"), b.alloc(K)
        run_layer(b, rg_layers[i % 2], xs[i], Y, ids, w, ws, THREE_KERNELS, W=RW, F=RF)
        ref.append((b.read(Y), b.read(ids)))
    outs = [(b.alloc(RW), b.alloc(K, "i32"), b.alloc(K)) for _ in range(n)]

    def sequence():
        for i in range(n):
            run_layer(b, rg_layers[i % 2], xs[i], *outs[i], ws, ALL, W=RW, F=RF)

    def check(tag):
        for i in range(n):
            assert np.array_equal(bits(b.read(outs[i][0])), bits(ref[i][0])), (tag, i)
            assert np.array_equal(b.read(outs[i][1]), ref[i][1]), (tag, i)
        for o in outs:
            b.zero(o[0])

    sequence()
    check("eager")
    b.graph_begin()
    sequence()
    gid = b.graph_end()
    for rep in range(2):
        b.graph_launch(gid)
        b.sync()
        check("replay %d" % rep)
    b.graph_free(gid)
    assert b.info()["fusedDecodeFault"] == 0


@pytest.mark.parametrize("experts,topk", [(512, 4), (300, 10), (130, 7)])
def test_fused_2560_other_routing_shapes(backend, oracle, experts, topk):
    # Fewer experts and smaller top-k at the real geometry (hidden rows past
    # topk x 640 and down products of absent slots idle), against the oracle
    # and the three kernels.
    b = backend
    lay = wl.DeviceLayer(b, layer=9, width=RW, ff=RF, experts=experts, base_seed=wl.BASE_SEED + 1)
    X = b.alloc(RW, zero=False)
    b.synth_normal(X, RW, 4100 + experts + topk, wl.STREAM_INPUT, 1.0)
    ws = b.alloc_bytes(b.moe_workspace_bytes(1, RW, RF, experts, topk))
    Y, ids, w = b.alloc(RW), b.alloc(topk, "i32"), b.alloc(topk)
    Y3, ids3, w3 = b.alloc(RW), b.alloc(topk, "i32"), b.alloc(topk)
    run_layer(b, lay, X, Y, ids, w, ws, ALL, E=experts, K=topk, W=RW, F=RF)
    run_layer(b, lay, X, Y3, ids3, w3, ws, THREE_KERNELS, E=experts, K=topk, W=RW, F=RF)
    got_ids = b.read(ids)
    host = wl.host_layer(oracle, 9, width=RW, ff=RF, experts=experts, base_seed=wl.BASE_SEED + 1,
                         expert_ids=list(got_ids))
    eY, eids, ew = oracle.moe_layer(b.read(X), 1, host["Wr"], host["arena"], host["stride"], host["shared"],
                                    host["Wsg"], RW, RF, experts, topk)
    lay.free()
    assert np.array_equal(got_ids, eids)
    assert np.array_equal(bits(b.read(w)), bits(ew))
    got = b.read(Y)
    assert tol_ok(got, eY), float(np.abs(got - eY).max())
    assert np.array_equal(bits(got), bits(b.read(Y3)))
    assert b.info()["fusedDecodeFault"] == 0


@pytest.mark.parametrize("geometry", ["2048", "2560"])
def test_router_prefetch_changes_no_bits(backend, two_layers, rg_layers, geometry):
    # Each step names the next step's router matrix (sm_prefetch_router), so
    # the single launch pulls it into L2 while it waits: eager and replayed
    # from a graph, the bits equal those of the same steps without hints. A
    # hint whose buffer was freed before the call is dropped.
    b = backend
    E, K = wl.EXPERTS, wl.TOPK
    W, F, lays = (wl.WIDTH, wl.FF, two_layers) if geometry == "2048" else (RW, RF, rg_layers)
    n = 8
    xs = []
    for i in range(n):
        x = b.alloc(W, zero=False)
        b.synth_normal(x, W, 2100 + i, wl.STREAM_INPUT, 1.0)
        xs.append(x)
    ws = b.alloc_bytes(b.moe_workspace_bytes(1, W, F, E, K))
    outs = [(b.alloc(W), b.alloc(K, "i32"), b.alloc(K)) for _ in range(n)]

    def sequence(hint):
        for i in range(n):
            if hint:
                b.prefetch_router(lays[(i + 1) % 2].Wr, E, W)
            run_layer(b, lays[i % 2], xs[i], *outs[i], ws, ALL, W=W, F=F)

    sequence(False)
    ref = [(bits(b.read(o[0])), b.read(o[1])) for o in outs]

    def check(tag):
        for i in range(n):
            assert np.array_equal(bits(b.read(outs[i][0])), ref[i][0]), (tag, i)
            assert np.array_equal(b.read(outs[i][1]), ref[i][1]), (tag, i)
            b.zero(outs[i][0])

    sequence(True)
    check("eager")
    b.graph_begin()
    sequence(True)
    gid = b.graph_end()
    for rep in range(2):
        b.graph_launch(gid)
        b.sync()
        check("replay %d" % rep)
    b.graph_free(gid)
    gone = b.alloc(E * W, zero=True)
    b.prefetch_router(gone, E, W)
    b.free(gone)
    run_layer(b, lays[0], xs[0], *outs[0], ws, ALL, W=W, F=F)
    assert np.array_equal(bits(b.read(outs[0][0])), ref[0][0])
    assert b.info()["fusedDecodeFault"] == 0


def test_router_prefetch_rejects_bad_hints(backend, two_layers):
    b = backend
    with pytest.raises(sm.ArgumentError):
        b.prefetch_router(two_layers[0].Wr, 0, wl.WIDTH)
    with pytest.raises(sm.ArgumentError):
        b.prefetch_router(two_layers[0].Wr, wl.EXPERTS, 100)
    with pytest.raises(sm.StrataError):
        b.prefetch_router(two_layers[0].Wr, wl.EXPERTS * 2, wl.WIDTH)  # more rows than the buffer holds
    b.prefetch_router(None)


def test_fused_2560_give_up_reported_and_reset(backend, rg_layers):
    # The same forced give-up at the real geometry: NaN outputs, SM_E_FAULT
    # from sync, bit-identical results after the reset.
    b = backend
    E, K = wl.EXPERTS, wl.TOPK
    lay = rg_layers[0]
    X = b.alloc(RW, zero=False)
    b.synth_normal(X, RW, 37, wl.STREAM_INPUT, 1.0)
    ws = b.alloc_bytes(b.moe_workspace_bytes(1, RW, RF, E, K))
    ids, w = b.alloc(K, "i32"), b.alloc(K)
    Y0, Y1, Y2 = (b.alloc(RW) for _ in range(3))
    run_layer(b, lay, X, Y0, ids, w, ws, ALL, W=RW, F=RF)
    y0 = b.read(Y0)
    try:
        b.fused_test_hooks(spin_limit=64, withhold=True)
        print("fused 2560 give-up: withheld launch", flush=True)
        run_layer(b, lay, X, Y1, ids, w, ws, ALL, W=RW, F=RF)
        with pytest.raises(sm.StrataError) as err:
            b.idle()
        assert err.value.code == sm.SM_E_FAULT
    finally:
        b.fused_test_hooks()
        b.fused_reset()
    assert np.all(np.isnan(b.read(Y1)))
    run_layer(b, lay, X, Y2, ids, w, ws, ALL, W=RW, F=RF)
    assert np.array_equal(bits(b.read(Y2)), bits(y0))
    assert b.info()["fusedDecodeFault"] == 0
