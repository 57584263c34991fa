"""The MoE stage replayed from a HIP graph (sm_graph_begin / sm_graph_end /
sm_graph_launch): every replay must give the bits of the same call issued
directly. Each path is covered (decode, batched decode, the small-batch and
the full prefill path with its second stream, and the block entry), with the
program's own eager work and synchronisations between the replays."""
import numpy as np
import pytest

from stratacuda_amd import workload as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def layers(backend):
    ls = [wl.DeviceLayer(backend, layer=l) for l in range(2)]
    yield ls
    for l in ls:
        l.free()


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("tokens", [1, 4, 8, 20, 40, 512])
@pytest.mark.parametrize("block", [False, True])
def test_graph_replay_matches_eager(backend, layers, tokens, block):
    b = backend
    W, F, E, K = wl.WIDTH, wl.FF, wl.EXPERTS, wl.TOPK
    lay, other = layers
    X, X2 = b.alloc(tokens * W, zero=False), b.alloc(tokens * W, zero=False)
    b.synth_normal(X, tokens * W, 900 + tokens, wl.STREAM_INPUT, 1.0)
    b.synth_normal(X2, tokens * W, 950 + tokens, wl.STREAM_INPUT, 1.0)
    Y, Y2 = b.alloc(tokens * W), b.alloc(tokens * W)
    ids, w = b.alloc(tokens * K, "i32"), b.alloc(tokens * K)
    ids2, w2 = b.alloc(tokens * K, "i32"), b.alloc(tokens * K)
    if block:
        nbytes = b.moe_block_workspace_bytes(tokens, W, F, E, K)
    else:
        nbytes = b.moe_workspace_bytes(tokens, W, F, E, K)
    ws, ws2 = b.alloc_bytes(nbytes), b.alloc_bytes(nbytes)

    def call(x, y, i, wt, work, l):
        if block:
            b.moe_block(x, tokens, l.gamma, 1e-6, l.Wr, l.arena, l.stride, l.shared, l.Wsg, W, F, E, K, y, i, wt,
                        work)
        else:
            b.moe_layer(x, tokens, l.Wr, l.arena, l.stride, l.shared, l.Wsg, W, F, E, K, y, i, wt, work)

    call(X, Y, ids, w, ws, lay)
    b.sync()
    ey, eids, ew = b.read(Y), b.read(ids), b.read(w)
    assert np.all(np.isfinite(ey))

    b.graph_begin()
    call(X, Y, ids, w, ws, lay)
    g = b.graph_end()
    try:
        for rep in range(4):
            # clobber the graph's outputs and workspace with other eager work first
            call(X2, Y, ids, w, ws, other)
            call(X2, Y2, ids2, w2, ws2, other)
            b.sync()
            b.graph_launch(g)
            b.sync()
            assert np.array_equal(b.read(ids), eids), "replay %d" % rep
            assert np.array_equal(bits(b.read(w)), bits(ew)), "replay %d" % rep
            assert np.array_equal(bits(b.read(Y)), bits(ey)), "replay %d" % rep
    finally:
        b.graph_free(g)


def test_capture_refuses_memsets_and_zero_fills_with_a_kernel(backend):
    """While a graph is being captured, a zero-filled allocation is refused
    and sm_zero records a fill kernel (no memset node): the replayed graph
    clears the words each time, including after eager writes between
    replays; a range that is not whole 32-bit words is refused."""
    import stratacuda_amd as sm
    b = backend
    buf = b.alloc(1000, "u32", zero=False)
    b.graph_begin()
    try:
        with pytest.raises(sm.ArgumentError):
            b.alloc(16, "f32", zero=True)
        with pytest.raises(sm.ArgumentError):
            b._check(sm.lib().sm_zero(b._ctx, buf.handle, 2, 8))
        b._check(sm.lib().sm_zero(b._ctx, buf.handle, 40, 400))  # words 10 .. 109
    finally:
        gid = b.graph_end()
    for rep in range(3):
        b.write(buf, np.full(1000, 0xA5A5A5A5 + rep, np.uint32))
        b.graph_launch(gid)
        got = b.read(buf)
        assert np.all(got[10:110] == 0), rep
        assert np.all(got[:10] == 0xA5A5A5A5 + rep) and np.all(got[110:] == 0xA5A5A5A5 + rep), rep
    b.graph_free(gid)
    b.free(buf)
