"""The allocation-free decode entry (sm_moe_layer_static) through the C ABI
against sm_moe_layer with a workspace, on two calls in a row, the second with
fewer tokens: up to 6 tokens both run the decode kernels and give the same
bits; from 7 to 16 tokens sm_moe_layer runs the grouped GEMMs, so the routing
(IDs and weights) is the same bits and the outputs agree within
1e-4 + 1e-3 |e|. It allocates nothing, and it refuses shapes beyond its
static scratch with a clear error."""
import numpy as np
import pytest

import stratacuda_amd as sm
from conftest import tol_ok
from stratacuda_amd import workload as wl

DECODE_BATCH_MAX = 6  # sm_moe_layer runs the decode kernels up to here

pytestmark = pytest.mark.gpu


def bits(a):
    return np.asarray(a).view(np.uint32)


@pytest.fixture(scope="module")
def layers(backend):
    made = {}
    yield made
    for lay in made.values():
        lay.free()


def _layer(backend, layers, width, ff):
    if (width, ff) not in layers:
        layers[(width, ff)] = wl.DeviceLayer(backend, layer=3, width=width, ff=ff)
    return layers[(width, ff)]


@pytest.mark.parametrize("width,ff,token_seq", [(2048, 512, (8, 1)), (2048, 512, (16, 3)), (2048, 512, (6, 2)),
                                                (2560, 640, (5, 1))])
def test_static_entry_matches_workspace_entry(backend, layers, width, ff, token_seq):
    b = backend
    E, K = wl.EXPERTS, wl.TOPK
    lay = _layer(b, layers, width, ff)
    Tmax = max(token_seq)
    X = b.alloc(Tmax * width, zero=False)
    Y_ref, Y = b.alloc(Tmax * width), b.alloc(Tmax * width)
    ids_ref, ids = b.alloc(Tmax * K, "i32"), b.alloc(Tmax * K, "i32")
    w_ref, w = b.alloc(Tmax * K), b.alloc(Tmax * K)
    ws = b.alloc_bytes(b.moe_workspace_bytes(Tmax, width, ff, E, K))
    for call, T in enumerate(token_seq):
        print("static entry: width %d ff %d call %d tokens %d" % (width, ff, call, T), flush=True)
        b.synth_normal(X, T * width, 4242 + 17 * call + T, wl.STREAM_INPUT, 1.0)
        b.moe_layer(X, T, lay.Wr, lay.arena, lay.stride, lay.shared, lay.Wsg, width, ff, E, K, Y_ref, ids_ref, w_ref,
                    ws)
        before = b.info()
        b.moe_layer_static(X, T, lay.Wr, lay.arena, lay.stride, lay.shared, lay.Wsg, width, ff, E, K, Y, ids, w)
        b.sync()
        after = b.info()
        assert after["allocatedBytes"] == before["allocatedBytes"] and after["buffers"] == before["buffers"]
        n, nk = T * width, T * K
        assert np.array_equal(b.read(ids, count=nk), b.read(ids_ref, count=nk)), (call, T)
        assert np.array_equal(bits(b.read(w, count=nk)), bits(b.read(w_ref, count=nk))), (call, T)
        got, want = b.read(Y, count=n), b.read(Y_ref, count=n)
        assert np.all(np.isfinite(got))
        if T <= DECODE_BATCH_MAX:
            assert np.array_equal(bits(got), bits(want)), (call, T, float(np.abs(got - want).max()))
        else:
            assert tol_ok(got, want), (call, T, float(np.abs(got - want).max()))
    for buf in (X, Y_ref, Y, ids_ref, ids, w_ref, w, ws):
        b.free(buf)


def test_static_entry_refuses_what_does_not_fit(backend, layers):
    b = backend
    E, K = wl.EXPERTS, wl.TOPK
    lay = _layer(b, layers, 2048, 512)
    X, Y = b.alloc(17 * 2048), b.alloc(17 * 2048)
    ids, w = b.alloc(17 * K, "i32"), b.alloc(17 * K)
    with pytest.raises(sm.ArgumentError, match="at most 16 tokens"):
        b.moe_layer_static(X, 17, lay.Wr, lay.arena, lay.stride, lay.shared, lay.Wsg, 2048, 512, E, K, Y, ids, w)
    # 16 tokens of ff 3072 need 2.2 MiB of decode scratch: beyond the 2 MiB array
    with pytest.raises(sm.ArgumentError, match="static scratch holds"):
        b.moe_layer_static(X, 16, lay.Wr, lay.arena, lay.stride, lay.shared, lay.Wsg, 2048, 3072, E, K, Y, ids, w)
    for buf in (X, Y, ids, w):
        b.free(buf)


def test_static_entry_orders_calls_from_two_contexts(backend, layers):
    """Two contexts on one GPU (two streams) call the allocation-free entry
    back to back without synchronising in between: each call waits for the
    previous one on the other stream, so every result equals the same call
    made alone."""
    b1 = backend
    b2 = sm.Backend(0)
    E, K, W, F, T = wl.EXPERTS, wl.TOPK, 2048, 512, 4
    try:
        lay1 = _layer(b1, layers, W, F)
        lay2 = wl.DeviceLayer(b2, layer=5)
        X1, X2 = b1.alloc(T * W, zero=False), b2.alloc(T * W, zero=False)
        b1.synth_normal(X1, T * W, 901, wl.STREAM_INPUT, 1.0)
        b2.synth_normal(X2, T * W, 902, wl.STREAM_INPUT, 1.0)
        out1 = [b1.alloc(T * W), b1.alloc(T * K, "i32"), b1.alloc(T * K)]
        out2 = [b2.alloc(T * W), b2.alloc(T * K, "i32"), b2.alloc(T * K)]

        def call1():
            b1.moe_layer_static(X1, T, lay1.Wr, lay1.arena, lay1.stride, lay1.shared, lay1.Wsg, W, F, E, K, *out1)

        def call2():
            b2.moe_layer_static(X2, T, lay2.Wr, lay2.arena, lay2.stride, lay2.shared, lay2.Wsg, W, F, E, K, *out2)

        def read(b, out):
            return [bits(b.read(o)) if o is out[0] or o is out[2] else b.read(o) for o in out]

        call1()
        b1.sync()
        want1 = read(b1, out1)
        call2()
        b2.sync()
        want2 = read(b2, out2)
        for rep in range(8):
            print("static entry, two contexts: round %d" % rep, flush=True)
            call1()
            call2()
            b1.sync()
            b2.sync()
            for got, want in zip(read(b1, out1), want1):
                assert np.array_equal(got, want), ("context 1", rep)
            for got, want in zip(read(b2, out2), want2):
                assert np.array_equal(got, want), ("context 2", rep)
        for buf in [X1] + out1:
            b1.free(buf)
        lay2.free()
    finally:
        b2.dispose()
