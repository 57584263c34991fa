"""Pack files on the CPU: the writer's layout against the reference's blob
layout and PackStore's checks (src/model.js:82-103, :160-167). The device
load (sm_load_experts) is tested in tests/test_gpu_pack.py."""
import json
import os

import numpy as np
import pytest

from stratacuda_amd import workload as wl

W, F, E = 128, 64, 16


@pytest.fixture(scope="module")
def layers(oracle):
    return [wl.host_layer(oracle, l, W, F, E, 11) for l in range(2)]


def test_pack_layout_is_the_arena(tmp_path, layers):
    man = wl.write_pack(str(tmp_path), W, F, E, 4, layers)
    raw = np.fromfile(os.path.join(str(tmp_path), "experts.bin"), np.uint8)
    bb = man["experts"]["blob_bytes"]
    assert bb == wl.blob_bytes(W, F)
    # vendor/strata/tools/pack_layer.py:54-65: the four planes in order
    assert man["experts"]["offsets"] == {"gate_up_codes": 0, "down_codes": 2 * F * W // 4,
                                         "gate_up_scales": 2 * F * W // 4 + W * F // 4,
                                         "down_scales": 2 * F * W // 4 + W * F // 4 + 2 * F * (W // 64) * 2}
    for l, lay in enumerate(layers):
        off = man["experts"]["layers"][l]["offset"]
        for e in (0, 7, E - 1):
            assert np.array_equal(raw[off + e * bb:off + (e + 1) * bb], lay["arena"][e * lay["stride"]:][:bb])
        soff = man["experts"]["shared"][l]["offset"]
        assert np.array_equal(raw[soff:soff + bb], lay["shared"][:bb])
    r = wl.PackReader(str(tmp_path))
    assert (r.width, r.ff, r.experts, r.layers) == (W, F, E, 2)
    assert np.array_equal(r.dense(1, "ffn_norm.weight"), layers[1]["gamma"])


def _edit(path, fn):
    m = json.load(open(os.path.join(path, "manifest.json")))
    fn(m)
    json.dump(m, open(os.path.join(path, "manifest.json"), "w"))


@pytest.mark.parametrize("case,match", [
    ("format", "canonical pack"), ("source", "requires Q2_0"), ("size", "size differs"),
    ("plane", "Invalid plane"), ("layout", "blob layout"), ("nonfinite", "Non-finite model weights")])
def test_pack_reader_rejects(tmp_path, layers, case, match):
    p = str(tmp_path)
    wl.write_pack(p, W, F, E, 4, layers)
    if case == "format":
        _edit(p, lambda m: m.update(format="strata-webcuda-v0"))
    elif case == "source":
        _edit(p, lambda m: m["experts"].update(source_type="IQ4_NL"))
    elif case == "size":
        with open(os.path.join(p, "experts.bin"), "ab") as f:
            f.write(b"\0")
    elif case == "plane":
        _edit(p, lambda m: m["tensors"]["blk.1.ffn_norm.weight"]["values"].update(offset=10 ** 9))
    elif case == "layout":
        _edit(p, lambda m: m["experts"].update(blob_bytes=m["experts"]["blob_bytes"] + 16))
    else:
        t = json.load(open(os.path.join(p, "manifest.json")))["tensors"]["blk.0.ffn_norm.weight"]
        with open(os.path.join(p, "dense.bin"), "r+b") as f:
            f.seek(t["values"]["offset"] + 8)
            f.write(np.array([np.inf], np.float32).tobytes())
    with pytest.raises(ValueError, match=match):
        r = wl.PackReader(p)
        r.dense(0, "ffn_norm.weight")
