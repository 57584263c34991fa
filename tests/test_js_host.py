"""The JavaScript host (stratacuda_amd/src: backend.js, ops.js,
residency.js, store.js, moe.js) under Node, through the Node-API addon.

CPU: tests/js/host_cpu.test.js over a stand-in addon (validation and error
conventions of src/backend.js:6-56, argument packing, buffer bookkeeping,
resident layout, kernel offsets) and tests/js/engine_cpu.test.js (the
session: plan.js / interpreter.js / engine.js launch structure and rules). GPU: tests/js/host_gpu.test.js runs the MoE
stage fused and host-driven on seeded layers; the expected routing and
outputs come from the CPU oracle, computed here and handed over as files."""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from stratacuda_amd import workload as wl

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
JS = os.path.join(ROOT, "tests", "js")
ADDON = os.path.join(ROOT, "stratacuda_amd", "src", "strata_addon.node")


def node_or_skip():
    node = shutil.which("node")
    if node is None:
        pytest.skip("node is not installed")
    if not os.path.exists(ADDON):
        pytest.fail("the Node-API addon is not built (run __graft_entry__.build())")
    return node


def run_node(script, *args, timeout=600):
    r = subprocess.run([node_or_skip(), os.path.join(JS, script)] + list(args), cwd=ROOT, stdout=subprocess.PIPE,
                       stderr=subprocess.STDOUT, text=True, timeout=timeout)
    print(r.stdout)
    assert r.returncode == 0, r.stdout[-4000:]
    return r.stdout


def test_js_host_cpu():
    out = run_node("host_cpu.test.js", timeout=120)
    assert "FAIL" not in out


def test_js_engine_cpu():
    # The session over the stand-in addon: program shape gate, one-token vs
    # batch launches, chunk bookkeeping, session rules and checkpoints.
    out = run_node("engine_cpu.test.js", timeout=120)
    assert "FAIL" not in out


def _case(oracle, tmp, name, width, ff, experts, topk, base_seed, tokens, input_seed, check_rows=None,
          host_driven=True):
    x = oracle.synth_normal(tokens * width, input_seed, wl.STREAM_INPUT, 1.0)
    full_layer = experts == wl.EXPERTS and width == wl.WIDTH
    if full_layer:
        seed = wl.layer_seed(0, base_seed)
        Wr = oracle.synth_normal(experts * width, seed, wl.STREAM_ROUTER, wl.ROUTER_SIGMA)
        logits = oracle.project(x, Wr, width, experts, tokens)
        ids, w = oracle.router(logits, experts, topk, tokens)
        rows = list(range(tokens)) if check_rows is None else check_rows
        sub = ids.reshape(tokens, topk)[rows].reshape(-1)
        host = wl.host_layer(oracle, 0, width, ff, experts, base_seed, expert_ids=sub)
        xs = x.reshape(tokens, width)[rows].reshape(-1)
        y, eids, _ = oracle.moe_layer(xs, len(rows), host["Wr"], host["arena"], host["stride"], host["shared"],
                                      host["Wsg"], width, ff, experts, topk)
        assert np.array_equal(eids, sub)
    else:
        host = wl.host_layer(oracle, 0, width, ff, experts, base_seed)
        y, ids, w = oracle.moe_layer(x, tokens, host["Wr"], host["arena"], host["stride"], host["shared"],
                                     host["Wsg"], width, ff, experts, topk)
        rows = None
    ids.astype(np.int32).tofile(os.path.join(tmp, name + "_ids.bin"))
    w.astype(np.float32).tofile(os.path.join(tmp, name + "_w.bin"))
    y.astype(np.float32).tofile(os.path.join(tmp, name + "_y.bin"))
    return {"name": name, "width": width, "ff": ff, "experts": experts, "topK": topk, "baseSeed": base_seed,
            "tokens": tokens, "inputSeed": input_seed, "checkRows": rows if check_rows is not None else [],
            "hostDriven": host_driven}


@pytest.mark.gpu
def test_js_host_gpu(oracle, tmp_path):
    tmp = str(tmp_path)
    cases = [
        _case(oracle, tmp, "small_decode", 128, 64, 16, 4, 11, 1, 101),
        _case(oracle, tmp, "small_prompt", 128, 64, 16, 4, 11, 37, 102),
        _case(oracle, tmp, "full_decode", wl.WIDTH, wl.FF, wl.EXPERTS, wl.TOPK, wl.BASE_SEED, 1, 103),
        _case(oracle, tmp, "full_prompt64", wl.WIDTH, wl.FF, wl.EXPERTS, wl.TOPK, wl.BASE_SEED, 64, 104,
              check_rows=[0, 17, 63]),
    ]
    json.dump({"cases": cases}, open(os.path.join(tmp, "manifest.json"), "w"))
    out = run_node("host_gpu.test.js", tmp)
    assert "FAIL" not in out


def _small_pack(oracle, path, tokens):
    W, F, E, K = 128, 64, 16, 4
    hosts = [wl.host_layer(oracle, l, W, F, E, 11) for l in range(2)]
    wl.write_pack(path, W, F, E, K, hosts)
    x = np.random.default_rng(tokens).normal(0, 1, tokens * W).astype(np.float32)
    h = hosts[1]
    y, ids, _ = oracle.moe_layer(x, tokens, h["Wr"], h["arena"], h["stride"], h["shared"], h["Wsg"], W, F, E, K)
    x.tofile(os.path.join(path, "x.bin"))
    ids.astype(np.int32).tofile(os.path.join(path, "ids.bin"))
    y.astype(np.float32).tofile(os.path.join(path, "y.bin"))


def test_js_pack_store_cpu(oracle, tmp_path):
    _small_pack(oracle, str(tmp_path), 1)
    out = run_node("pack.test.js", str(tmp_path), "cpu", timeout=120)
    assert "FAIL" not in out


@pytest.mark.gpu
@pytest.mark.parametrize("tokens", [1, 29])
def test_js_pack_store_gpu(oracle, tmp_path, tokens):
    # The extra files (x.bin, ids.bin, y.bin) are not in the manifest's file list.
    _small_pack(oracle, str(tmp_path), tokens)
    out = run_node("pack.test.js", str(tmp_path), "gpu", timeout=300)
    assert "FAIL" not in out
