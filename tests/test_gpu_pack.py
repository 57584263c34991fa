"""Loading a pack's experts into the resident arena on the GPU
(sm_load_experts through the C ABI): the loaded arena equals the file's bytes,
a layer run from it matches the CPU oracle (routing bit-exact, outputs within
|a - e| <= 1e-4 + 1e-3 |e|), non-finite fp16 scales are rejected naming the
first bad blob (src/model.js:164-165), and out-of-range reads are errors."""
import os
import time

import numpy as np
import pytest

import stratacuda_amd as sm
from conftest import tol_ok
from stratacuda_amd import workload as wl

pytestmark = pytest.mark.gpu


def run_layer(backend, lay, X, tokens, W, F, E, K):
    Y, ids, w = backend.alloc(tokens * W), backend.alloc(tokens * K, "i32"), backend.alloc(tokens * K)
    ws = backend.alloc_bytes(backend.moe_workspace_bytes(tokens, W, F, E, K))
    backend.moe_layer(X, tokens, lay.Wr, lay.arena, lay.stride, lay.shared, lay.Wsg, W, F, E, K, Y, ids, w, ws)
    return backend.read(Y), backend.read(ids), backend.read(w)


@pytest.mark.parametrize("tokens", [1, 37])
def test_layer_from_pack_small(backend, oracle, tmp_path, tokens):
    W, F, E, K = 128, 64, 16, 4
    hosts = [wl.host_layer(oracle, l, W, F, E, 11) for l in range(2)]
    wl.write_pack(str(tmp_path), W, F, E, K, hosts)
    r = wl.PackReader(str(tmp_path))
    lay = r.load_layer(backend, 1)
    h = hosts[1]
    assert np.array_equal(backend.read_bytes(lay.arena), h["arena"])
    assert np.array_equal(backend.read_bytes(lay.shared), h["shared"])
    x = np.random.default_rng(tokens).normal(0, 1, tokens * W).astype(np.float32)
    y, ids, w = run_layer(backend, lay, backend.alloc(x), tokens, W, F, E, K)
    ey, eids, ew = oracle.moe_layer(x, tokens, h["Wr"], h["arena"], h["stride"], h["shared"], h["Wsg"], W, F, E, K)
    assert np.array_equal(ids, eids)
    assert np.array_equal(w.view(np.uint32), ew.view(np.uint32))
    assert tol_ok(y, ey)
    lay.free()


def test_pack_rejects_nonfinite_scales_and_bad_ranges(backend, oracle, tmp_path):
    W, F, E = 128, 64, 16
    h = wl.host_layer(oracle, 0, W, F, E, 11)
    man = wl.write_pack(str(tmp_path), W, F, E, 4, [h])
    f = os.path.join(str(tmp_path), "experts.bin")
    bb, so = man["experts"]["blob_bytes"], man["experts"]["offsets"]["gate_up_scales"]
    arena = backend.alloc_bytes(wl.blob_stride(W, F) * E)
    backend.load_experts(f, 0, bb, E, arena, wl.blob_stride(W, F), so)
    # a NaN scale in blob 9's down plane and an inf in blob 12's gate/up plane
    raw = bytearray(open(f, "rb").read())
    at = 9 * bb + man["experts"]["offsets"]["down_scales"] + 6
    raw[at:at + 2] = np.array([0x7e00], np.uint16).tobytes()
    at = 12 * bb + so + 2
    raw[at:at + 2] = np.array([0xfc00], np.uint16).tobytes()
    bad = os.path.join(str(tmp_path), "bad.bin")
    open(bad, "wb").write(bytes(raw))
    with pytest.raises(sm.ArgumentError, match=r"Non-finite expert scales \(blob 9\)"):
        backend.load_experts(bad, 0, bb, E, arena, wl.blob_stride(W, F), so)
    with pytest.raises(sm.ArgumentError, match=r"Non-finite expert scales \(blob 2\)"):  # blobs 10..13 loaded
        backend.load_experts(bad, 10 * bb, bb, 4, arena, wl.blob_stride(W, F), so)
    with pytest.raises(sm.ArgumentError, match="out of bounds"):  # the file holds E + 1 blobs
        backend.load_experts(f, 2 * bb, bb, E, arena, wl.blob_stride(W, F), so)
    with pytest.raises(sm.ArgumentError, match="model file"):
        backend.load_experts(f + ".missing", 0, bb, 1, arena, wl.blob_stride(W, F), so)
    with pytest.raises(sm.StrataError):  # arena too small for the count
        backend.load_experts(f, 0, bb, E, backend.alloc_bytes(bb * 4), wl.blob_stride(W, F), so)


def test_full_layer_from_pack(backend, oracle, tmp_path):
    # One full-geometry layer (512 blobs of 884,736 bytes, 453 MB) written by
    # the host generator, streamed into HBM, compared with the device
    # generator's copy of the same layer, then run at T=1.
    W, F, E, K = wl.WIDTH, wl.FF, wl.EXPERTS, wl.TOPK
    h = wl.host_layer(oracle, 0)
    wl.write_pack(str(tmp_path), W, F, E, K, [h])
    r = wl.PackReader(str(tmp_path))
    t0 = time.perf_counter()
    lay = r.load_layer(backend, 0)
    backend.sync()
    dt = time.perf_counter() - t0
    print("loaded %.1f MB in %.3f s (%.2f GB/s from the page cache)" % (E * r.blob_bytes / 1e6, dt,
                                                                        E * r.blob_bytes / dt / 1e9))
    ref = wl.DeviceLayer(backend, 0)
    assert np.array_equal(backend.read_bytes(lay.arena), backend.read_bytes(ref.arena))
    x = backend.alloc(W, zero=False)
    backend.synth_normal(x, W, 404, wl.STREAM_INPUT, 1.0)
    y1, ids1, w1 = run_layer(backend, lay, x, 1, W, F, E, K)
    y2, ids2, w2 = run_layer(backend, ref, x, 1, W, F, E, K)
    assert np.array_equal(ids1, ids2) and np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    lay.free()
    ref.free()
