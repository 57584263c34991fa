"""The C-ABI library loads and exports every entry point the public header
declares; its kernel table mirrors the reference's parameter lists. CPU only:
nothing here initialises a GPU."""
import ctypes
import os
import re
import subprocess
import sys

import pytest

from conftest import REFERENCE, ROOT

HEADER = os.path.join(ROOT, "include", "strata_mi355x.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(sm_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    import stratacuda_amd as sm
    path = sm.LIB_PATH
    assert os.path.exists(path), "build first"
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (sm_\w+)", out))
    missing = [f for f in declared_functions() if f not in exported]
    assert not missing, missing
    lib = ctypes.CDLL(path)
    for f in declared_functions():
        getattr(lib, f)


def test_fused_decode_selection_rule():
    # The single-launch decode layer needs 256 blocks resident at once, one
    # per CU: a whole MI355X (256 CUs) qualifies; its DPX / CPX partitions
    # (128 / 32 CUs per partition), fewer CUs or no occupancy do not.
    import stratacuda_amd as sm
    L = sm.lib()
    assert L.sm_fused_fits(256, 1) == 1
    assert L.sm_fused_fits(304, 1) == 1
    assert L.sm_fused_fits(128, 2) == 1
    for cus, per_cu in [(255, 1), (128, 1), (32, 1), (256, 0), (0, 4), (-1, 1)]:
        assert L.sm_fused_fits(cus, per_cu) == 0, (cus, per_cu)


def test_library_contains_gfx950_code_object():
    import stratacuda_amd as sm
    data = open(sm.LIB_PATH, "rb").read()
    assert b"gfx950" in data


def test_kernel_table_lists_reference_kernels():
    import stratacuda_amd as sm
    sigs = sm.kernel_signatures()
    for name in ["strata_project", "strata_router", "strata_router_batch", "strata_q2_gate_up", "strata_q2_down",
                 "strata_moe_combine", "strata_moe_combine_batch", "strata_gather_rows", "strata_scatter_rows",
                 "strata_unpack_half", "strata_expert_scales", "strata_q2_project", "strata_quant_project",
                 "strata_norm", "strata_elementwise", "strata_gemv",
                 # the fixture model's kernels outside the MoE path
                 "strata_embedding", "strata_rope_frequencies", "strata_rope_table", "strata_rope_position",
                 "strata_hc_mix", "strata_hc_write", "strata_conv", "strata_gdn_gates", "strata_gdn_step",
                 "strata_slice", "strata_kv_append", "strata_attention", "strata_attention_gate", "strata_ple_gate",
                 "strata_ple_broadcast", "strata_ple_add", "strata_argmax", "strata_bf16_project",
                 "strata_quant_gemv", "strata_ple_decode", "strata_embed", "strata_rope"]:
        assert name in sigs, name


@pytest.mark.skipif(not os.path.exists(os.path.join(REFERENCE, "kernels", "strata.cu")),
                    reason="reference tree not present")
def test_kernel_signatures_match_reference_source():
    # Parameter names and order as in the reference's kernels/strata.cu: the
    # JavaScript host maps named arguments by these names (compile.mjs:55).
    import stratacuda_amd as sm
    src = open(os.path.join(REFERENCE, "kernels", "strata.cu")).read()
    types = {"float*": "f32*", "unsignedint*": "u32*", "int*": "i32*", "int": "i32", "float": "f32"}
    for name, params in sm.kernel_signatures().items():
        m = re.search(r"__global__\s+void\s+" + name + r"\s*\(([^)]*)\)", src)
        assert m, name
        ref = []
        for p in m.group(1).split(","):
            p = p.replace("const", "").strip()
            pname = re.findall(r"\w+$", p)[0]
            ptype = re.sub(r"\s+", "", p[:-len(pname)])
            ref.append((pname, types[ptype]))
        assert params == ref, (name, params, ref)


def test_backend_fails_loudly_without_gpu():
    # The product path has no CPU fallback: constructing a backend on a host
    # without a usable GPU raises.
    code = ("import sys; sys.path.insert(0, %r)\n"
            "import stratacuda_amd as sm\n"
            "try:\n    sm.Backend(0)\nexcept Exception as e:\n    print('raised', type(e).__name__)\n"
            "else:\n    print('no-error')\n") % ROOT
    env = dict(os.environ, HIP_VISIBLE_DEVICES="-1", ROCR_VISIBLE_DEVICES="-1")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120, env=env)
    assert "raised StrataError" in r.stdout, r.stdout + r.stderr
