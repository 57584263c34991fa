"""The fused MoE path at the real model's geometry (src/model.js:4-6: hidden
2560, expert ff 640, 512 experts, top-10 + shared, Q2 blobs of 1,382,400
bytes) on the GPU against the CPU oracle: routed IDs and routing weights
bit-exact for every token, outputs of all (or a sample of) tokens within
|a - e| <= 1e-4 + 1e-3 |e|. The same kernels run both geometries; these
cases cover the decode kernels with and without a token dimension, the
16-row tiles of small batches and the 64-row tiles of prompts."""
import numpy as np
import pytest

from conftest import tol_ok
from stratacuda_amd import workload as wl

pytestmark = pytest.mark.gpu

W, F, E, K = 2560, 640, 512, 10


@pytest.fixture(scope="module")
def real_layer(backend):
    layer = wl.DeviceLayer(backend, layer=0, width=W, ff=F, experts=E, base_seed=wl.BASE_SEED + 1)
    yield layer
    layer.free()


def test_real_blob_layout(real_layer):
    assert wl.blob_bytes(W, F) == 1382400
    assert real_layer.stride >= 1382400 and real_layer.stride % 256 == 0


@pytest.mark.parametrize("tokens,bias,sample", [(1, False, 1), (1, True, 1), (8, False, 8), (24, False, 6),
                                                (40, False, 6), (512, False, 12), (2048, True, 12)])
def test_real_geometry_layer(backend, oracle, real_layer, tokens, bias, sample):
    layer = real_layer
    X = backend.alloc(tokens * W, "f32", zero=False)
    backend.synth_normal(X, tokens * W, layer.seed + 500 + tokens, wl.STREAM_INPUT, 1.0)
    b = wl.zipf_bias(E, layer.seed) if bias else None
    Y, ids, w = backend.alloc(tokens * W), backend.alloc(tokens * K, "i32"), backend.alloc(tokens * K)
    ws = backend.alloc_bytes(backend.moe_workspace_bytes(tokens, W, F, E, K))
    backend.moe_layer(X, tokens, layer.Wr, layer.arena, layer.stride, layer.shared, layer.Wsg, W, F, E, K, Y, ids, w,
                      ws, bias=backend.alloc(b) if bias else None)
    got_y, got_ids, got_w, xh = backend.read(Y), backend.read(ids), backend.read(w), backend.read(X)
    assert np.all(np.isfinite(got_y))
    logits = oracle.project(xh, backend.read(layer.Wr), W, E, tokens)
    if bias:
        logits = (logits.reshape(tokens, E) + b).reshape(-1)
    rids, rw = oracle.router(logits, E, K, tokens)
    assert np.array_equal(got_ids, rids)
    assert np.array_equal(got_w.view(np.uint32), rw.view(np.uint32))
    rng = np.random.default_rng(tokens)
    pick = np.sort(rng.choice(tokens, min(sample, tokens), replace=False))
    sub_ids = got_ids.reshape(tokens, K)[pick].reshape(-1)
    host = wl.host_layer(oracle, 0, width=W, ff=F, experts=E, base_seed=wl.BASE_SEED + 1, expert_ids=sub_ids)
    xs = xh.reshape(tokens, W)[pick].reshape(-1)
    eY, eids, _ = oracle.moe_layer(xs, len(pick), host["Wr"], host["arena"], host["stride"], host["shared"],
                                   host["Wsg"], W, F, E, K, bias=b)
    assert np.array_equal(eids, sub_ids)
    gy = got_y.reshape(tokens, W)[pick].reshape(-1)
    assert tol_ok(gy, eY), "max abs err %g" % np.abs(gy - eY).max()
