"""The config-1 fixture through the JavaScript host: the reference's untrained
4-layer model (createFixture(1234)) decoded by StrataEngine over the HIP
backend, against the CPU oracle's restatement of the same decode.

CPU: the JavaScript generator (stratacuda_amd/src/fixture.js) and n-gram rows
(stratacuda_amd/src/model.js) equal the oracle's (oracle/fixture.py) bit for
bit. GPU: tests/js/fixture_gpu.test.js checks the reference's known answers
and the session API on the device and traces 16 seeded tokens; routed expert
IDs and argmax tokens must equal the oracle's, logits are compared bit for bit
(every kernel keeps the reference's f32 order) and, as the stated bar, within
|a - e| <= 1e-4."""
import json
import os

import numpy as np
import pytest

from test_js_host import run_node


def test_js_fixture_generator_matches_oracle(oracle, tmp_path):
    from oracle import fixture as fx
    run_node("fixture_dump.js", str(tmp_path), "1234", timeout=120)
    index = json.load(open(os.path.join(str(tmp_path), "index.json")))
    values = np.fromfile(os.path.join(str(tmp_path), "values.bin"), dtype="<f4")
    model = fx.create_fixture(1234)
    assert index["config"] == {k: (int(v) if isinstance(v, float) and v.is_integer() else v)
                               for k, v in model.config.items()}
    assert [t["name"] for t in index["tensors"]] == list(model.tensors)
    at = 0
    for t in index["tensors"]:
        want = model.data(t["name"])
        assert t["shape"] == model.shape(t["name"]), t["name"]
        assert np.array_equal(values[at:at + want.size].view(np.uint32), want.view(np.uint32)), t["name"]
        at += want.size
    assert at == values.size
    rows = []
    for prev in ([], [3], [5, 9], [39, 9], [9, 39]):
        for token in range(model.config["vocab"]):
            rows.append(fx.ngram_rows(token, prev, model.constants, model.config["eos"]))
    assert index["ngram"] == rows


@pytest.mark.gpu
def test_js_fixture_decode_on_gpu(oracle, tmp_path):
    from oracle import fixture as fx
    rng = np.random.default_rng(20261202)
    tokens = [int(t) for t in rng.integers(0, 40, 16)]
    json.dump({"tokens": tokens}, open(os.path.join(str(tmp_path), "request.json"), "w"))
    out = run_node("fixture_gpu.test.js", str(tmp_path), timeout=300)
    assert "FAIL" not in out
    trace = json.load(open(os.path.join(str(tmp_path), "trace.json")))
    e = fx.OracleEngine(fx.create_fixture(1234))
    worst, exact = 0.0, True
    for t, step in zip(tokens, trace["steps"]):
        tok, logits = e.step(t)
        assert step["routes"] == [r["ids"] for r in e.routes]
        assert step["token"] == tok
        got = np.array(step["logits"], np.uint32).view(np.float32)
        assert np.all(np.isfinite(got))
        worst = max(worst, float(np.max(np.abs(got.astype(np.float64) - logits))))
        exact = exact and np.array_equal(got.view(np.uint32), logits.view(np.uint32))
    print("fixture decode: 16 steps, max |logit - oracle| = %.3g, bit-exact: %s" % (worst, exact))
    assert worst <= 1e-4
    assert exact
    prompt = json.load(open(os.path.join(str(tmp_path), "prompt.json")))
    assert [p["chunkSize"] for p in prompt] == [1, 2, 5]
    for p in prompt:
        e = fx.OracleEngine(fx.create_fixture(1234))
        e.step(2, predict=False)
        tok, logits = fx.prefill(e, [7, 4, 8, 7, 4], chunk_size=p["chunkSize"])
        assert p["routes"] == [[r["position"], r["layer"], r["ids"]] for r in e.routes]
        assert p["token"] == tok
        same_bits(p["logits"], logits)
        tok, logits = e.step(8)
        assert p["nextToken"] == tok
        same_bits(p["next"], logits)
    print("fixture prompt chunks 1/2/5 + next decode: bit-exact with the oracle")


def same_bits(got_bits, want):
    got = np.array(got_bits, np.uint32)
    assert np.array_equal(got, np.asarray(want, np.float32).view(np.uint32)), \
        "max |diff| %g" % np.max(np.abs(got.view(np.float32).astype(np.float64) - want))
