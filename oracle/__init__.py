"""CPU oracle for the StrataCuda MoE path (ctypes over liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py``, always as the checker or the timed CPU
baseline, never as the product. ``strata_oracle.c`` restates each kernel of the
reference's ``kernels/strata.cu`` with its exact f32 operation order; its header
lists what pins each function.

Parity status: every function here is pinned (see the header of
``strata_oracle.c`` and tests/test_oracle_*.py).
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_DEQUANT = os.path.join(HERE, "_ref", "ref_dequant")

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_i = ctypes.c_int
_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_vp = ctypes.c_void_p

_lib = None


def build():
    """Compile liboracle.so (and oracle/_ref when the reference tree is present)."""
    subprocess.run(["make", "-s", "-B", "-C", HERE, "all"], check=True)
    if os.path.isdir("/root/reference/vendor/strata/include"):
        subprocess.run(["make", "-s", "-B", "-C", HERE, "ref"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("oracle/liboracle.so is not built; run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "or_half_bits": (ctypes.c_float, [ctypes.c_uint32]),
            "or_expf": (ctypes.c_float, [ctypes.c_float]),
            "or_sigmoid": (ctypes.c_float, [ctypes.c_float]),
            "or_unpack_half": (None, [_u32p, _f32p, _i]),
            "or_expert_scales": (None, [_u32p, _f32p, _i, _i]),
            "or_project": (None, [_f32p, _f32p, _f32p, _i, _i, _i, _i, _i]),
            "or_q2_gate_up": (None, [_f32p, _u32p, _vp, _vp, _f32p, _i, _i, _i, _i, _i, _i, _i]),
            "or_q2_down": (None, [_f32p, _u32p, _vp, _vp, _f32p, _i, _i, _i, _i, _i, _i, _i, _i]),
            "or_q2_project": (None, [_f32p, _u32p, _f32p, _i, _i, _i, _i, _i, _i, _i, _i, _i]),
            "or_quant_project": (None, [_f32p, _u32p, _f32p, _f32p, _f32p, _i, _i, _i, _i, _i, _i, _i,
                                        _i, _i, _i]),
            "or_norm": (None, [_f32p, _f32p, _f32p, _i, _i, _i, _i, ctypes.c_float, ctypes.c_float]),
            "or_elementwise": (None, [_f32p, _f32p, _f32p, _i, _i, ctypes.c_float]),
            "or_router_batch": (None, [_f32p, _i32p, _f32p, _i, _i, _i]),
            "or_moe_combine_batch": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _i, _i, _i]),
            "or_gather_rows": (None, [_f32p, _i32p, _f32p, _i, _i]),
            "or_scatter_rows": (None, [_f32p, _i32p, _f32p, _i, _i]),
            "or_dispatch": (_i, [_i32p, _i, _i, _i, _i32p, _i32p, _i32p, _i32p]),
            "or_moe_layer": (_i, [_f32p, _i, _f32p, _vp, _u8p, _i64, _u8p, _f32p, _i, _i, _i, _i, _f32p,
                                  _i32p, _f32p, _vp]),
            "or_set_threads": (None, [_i]),
            "or_max_threads": (_i, []),
            "or_moe_block": (_i, [_f32p, _f32p, _i, _f32p, _f32p, _u8p, _i64, _u8p, _f32p, _i, _i, _i,
                                  _i, _i32p, _f32p]),
            "or_rand": (_u64, [_u64, _u64, _u64]),
            "or_normal": (ctypes.c_double, [_u64, _u64, _u64]),
            "or_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "or_synth_normal": (None, [_f32p, _i64, _u64, _u64, ctypes.c_double]),
            "or_synth_uniform_pm": (None, [_f32p, _i64, _u64, _u64, ctypes.c_double]),
            "or_synth_blob": (None, [_u8p, _i, _i, _u64, _u64, ctypes.c_double]),
            "or_expf_survey": (None, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                      np.ctypeslib.ndpointer(dtype=np.uint64, flags="C_CONTIGUOUS")]),
            # strata_oracle_model.c: the fixture model's other kernels
            "or_logf": (ctypes.c_float, [ctypes.c_float]),
            "or_sinf": (ctypes.c_float, [ctypes.c_float]),
            "or_cosf": (ctypes.c_float, [ctypes.c_float]),
            "or_embedding": (None, [_vp, _vp, _vp, _vp, _f32p, _i, _i, _i, _i, _i, _i, _i, _i, _i]),
            "or_rope_frequencies": (None, [_f32p, _f32p, _i, ctypes.c_float]),
            "or_rope_table": (None, [_f32p, _f32p, _f32p, _f32p, _i, _i]),
            "or_rope_position": (None, [_f32p, _f32p, _f32p, _f32p, _i, _i, _i, _i, _i]),
            "or_hc_mix": (None, [_f32p, _f32p, _f32p, _i, _i]),
            "or_hc_write": (None, [_f32p, _f32p, _f32p, _i, _i]),
            "or_conv": (None, [_f32p, _f32p, _f32p, _f32p, _i, _i, _i, _i]),
            "or_gdn_gates": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _i]),
            "or_gdn_step": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _i, _i, _i]),
            "or_slice": (None, [_f32p, _f32p, _i, _i, _i, _i]),
            "or_kv_append": (None, [_f32p, _f32p, _f32p, _f32p, _i, _i]),
            "or_attention": (None, [_f32p, _f32p, _f32p, _i32p, _f32p, _i, _i, _i, _i, ctypes.c_float]),
            "or_attention_gate": (None, [_f32p, _f32p, _f32p, _i, _i]),
            "or_ple_gate": (None, [_f32p, _f32p, _f32p, _i, _i]),
            "or_ple_broadcast": (None, [_f32p, _f32p, _f32p, _i, _i]),
            "or_ple_add": (None, [_f32p, _f32p, _f32p, _i]),
            "or_argmax": (_i, [_f32p, _i]),
            "or_bf16_project": (None, [_f32p, _u32p, _f32p, _i, _i, _i, _i, _i]),
            "or_embed_batch": (None, [_f32p, _f32p, _i, _i, _i]),
            "or_hc_mix_batch": (None, [_f32p, _f32p, _f32p, _i, _i, _i]),
            "or_hc_write_batch": (None, [_f32p, _f32p, _f32p, _i, _i, _i]),
            "or_conv_batch": (None, [_f32p, _f32p, _f32p, _f32p, _i, _i, _i, _i, _i]),
            "or_gdn_gates_batch": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _i, _i]),
            "or_gdn_batch": (None, [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _i, _i, _i, _i]),
            "or_rope_batch": (None, [_f32p, _f32p, _f32p, _f32p, _i, _i, _i, _i]),
            "or_kv_append_batch": (None, [_f32p, _f32p, _f32p, _f32p, _i, _i, _i]),
            "or_attention_gate_batch": (None, [_f32p, _f32p, _f32p, _i, _i, _i]),
            "or_ple_broadcast_batch": (None, [_f32p, _f32p, _f32p, _i, _i, _i]),
            "or_attention_batch": (None, [_f32p, _f32p, _f32p, _f32p, _i, _i, _i, _i, ctypes.c_float, _i]),
            "or_ple_decode": (None, [_u32p, _f32p, _i]),
            "or_embed": (None, [_f32p, _f32p, _i, _i]),
            "or_rope": (None, [_f32p, _f32p, _f32p, _f32p, _i, _i, _i]),
            "or_math_survey": (None, [_i, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                      np.ctypeslib.ndpointer(dtype=np.uint64, flags="C_CONTIGUOUS")]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def u32(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


def i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


# ---------------------------------------------------------------- kernels
def half_bits(h):
    return lib().or_half_bits(int(h))


def expf(x):
    return np.float32(lib().or_expf(float(np.float32(x))))


def unpack_half(packed_u32, count):
    out = np.zeros(count, np.float32)
    lib().or_unpack_half(u32(packed_u32), out, count)
    return out


def expert_scales(blob_u32, offset, count):
    out = np.zeros(count, np.float32)
    lib().or_expert_scales(u32(blob_u32), out, offset, count)
    return out


def project(X, W, cols, rows, tokens, output_stride=None, output_offset=0, Y=None):
    output_stride = rows if output_stride is None else output_stride
    Y = np.zeros(tokens * output_stride, np.float32) if Y is None else Y
    lib().or_project(f32(X), f32(W), Y, cols, rows, tokens, output_stride, output_offset)
    return Y


def q2_gate_up(X, blob_u32, width, ff, tokens, mapping=None, scales=None, code_offset=0, scale_offset=0):
    hidden = np.zeros(tokens * ff, np.float32)
    m = None if mapping is None else i32(mapping)
    s = None if scales is None else f32(scales)
    lib().or_q2_gate_up(f32(X), u32(blob_u32), _ptr(s), _ptr(m), hidden, width, ff, tokens,
                        int(m is not None), int(s is not None), code_offset, scale_offset)
    return hidden


def q2_down(hidden, blob_u32, Y, width, ff, tokens, mapping=None, scales=None, output_offset=0,
            code_offset=0, scale_offset=0):
    m = None if mapping is None else i32(mapping)
    s = None if scales is None else f32(scales)
    lib().or_q2_down(f32(hidden), u32(blob_u32), _ptr(s), _ptr(m), Y, width, ff, tokens,
                     int(m is not None), int(s is not None), output_offset, code_offset, scale_offset)
    return Y


def q2_project(X, blob_u32, Y, cols, rows, tokens, output_stride, output_offset, code_offset, scale_offset,
               weight_row, row_stride):
    lib().or_q2_project(f32(X), u32(blob_u32), Y, cols, rows, tokens, output_stride, output_offset,
                        code_offset, scale_offset, weight_row, row_stride)
    return Y


def quant_project(X, codes, scales, offsets, Y, cols, rows, tokens, output_stride, output_offset, bits,
                  group_size, bias, codebook, has_offset):
    lib().or_quant_project(f32(X), u32(codes), f32(scales), f32(offsets), Y, cols, rows, tokens,
                           output_stride, output_offset, bits, group_size, bias, codebook, has_offset)
    return Y


def norm(X, W, cols, rows, weight_rows=1, mode=0, epsilon=1e-6, scale=1.0):
    Y = np.zeros(cols * rows, np.float32)
    lib().or_norm(f32(X), f32(W), Y, cols, rows, weight_rows, mode, epsilon, scale)
    return Y


def elementwise(A, B, mode, scale=1.0):
    A = f32(A)
    Y = np.zeros_like(A)
    lib().or_elementwise(A, f32(B), Y, A.size, mode, scale)
    return Y


def router(logits, experts, top_k, tokens=1):
    ids = np.zeros(tokens * top_k, np.int32)
    w = np.zeros(tokens * top_k, np.float32)
    lib().or_router_batch(f32(logits), ids, w, experts, top_k, tokens)
    return ids, w


def moe_combine(parts, weights, shared, shared_gate, width, count, tokens=1):
    Y = np.zeros(width * tokens, np.float32)
    lib().or_moe_combine_batch(f32(parts), f32(weights), f32(shared), f32(shared_gate), Y, width, count, tokens)
    return Y


def gather_rows(X, indices, width, rows):
    Y = np.zeros(width * rows, np.float32)
    lib().or_gather_rows(f32(X), i32(indices), Y, width, rows)
    return Y


def scatter_rows(X, indices, Y, width, rows):
    lib().or_scatter_rows(f32(X), i32(indices), Y, width, rows)
    return Y


def dispatch(ids, tokens, top_k, experts):
    offsets = np.zeros(experts + 1, np.int32)
    n = tokens * top_k
    rows = np.zeros(n, np.int32)
    parts = np.zeros(n, np.int32)
    where = np.zeros(n, np.int32)
    rc = lib().or_dispatch(i32(ids), tokens, top_k, experts, offsets, rows, parts, where)
    if rc:
        raise ValueError("dispatch failed (%d)" % rc)
    return offsets, rows, parts, where


def set_threads(n):
    """OpenMP threads for the oracle's parallel loops."""
    lib().or_set_threads(int(n))


def max_threads():
    return int(lib().or_max_threads())


def moe_layer(X, tokens, Wr, arena, blob_stride, shared_blob, Wsg, width, ff, experts, top_k, bias=None,
              want_logits=False):
    Y = np.zeros(tokens * width, np.float32)
    ids = np.zeros(tokens * top_k, np.int32)
    w = np.zeros(tokens * top_k, np.float32)
    logits = np.zeros(tokens * experts, np.float32) if want_logits else None
    b = None if bias is None else f32(bias)
    rc = lib().or_moe_layer(f32(X), tokens, f32(Wr), _ptr(b), np.ascontiguousarray(arena, np.uint8),
                            blob_stride, np.ascontiguousarray(shared_blob, np.uint8), f32(Wsg), width, ff,
                            experts, top_k, Y, ids, w, _ptr(logits))
    if rc:
        raise RuntimeError("or_moe_layer failed (%d)" % rc)
    return (Y, ids, w, logits) if want_logits else (Y, ids, w)


def moe_block(H, tokens, gamma, Wr, arena, blob_stride, shared_blob, Wsg, width, ff, experts, top_k):
    Hout = np.zeros(tokens * width, np.float32)
    ids = np.zeros(tokens * top_k, np.int32)
    w = np.zeros(tokens * top_k, np.float32)
    rc = lib().or_moe_block(f32(H), Hout, tokens, f32(gamma), f32(Wr), np.ascontiguousarray(arena, np.uint8),
                            blob_stride, np.ascontiguousarray(shared_blob, np.uint8), f32(Wsg), width, ff,
                            experts, top_k, ids, w)
    if rc:
        raise RuntimeError("or_moe_block failed (%d)" % rc)
    return Hout, ids, w


# ------------------------------------------------------- synthetic inputs
def blob_layout(width, ff):
    gu = 0
    dn = 2 * ff * width // 4
    gus = dn + width * ff // 4
    ds = gus + 2 * ff * (width // 64) * 2
    end = ds + width * (ff // 64) * 2
    return {"gate_up_codes": gu, "down_codes": dn, "gate_up_scales": gus, "down_scales": ds, "blob_bytes": end}


def synth_normal(n, seed, stream, sigma):
    out = np.zeros(n, np.float32)
    lib().or_synth_normal(out, n, seed, stream, sigma)
    return out


def synth_uniform_pm(n, seed, stream, amp):
    out = np.zeros(n, np.float32)
    lib().or_synth_uniform_pm(out, n, seed, stream, amp)
    return out


def synth_blob(width, ff, seed, stream, sigma=0.05):
    out = np.zeros(blob_layout(width, ff)["blob_bytes"], np.uint8)
    lib().or_synth_blob(out, width, ff, seed, stream, sigma)
    return out


def rand(seed, stream, i):
    return lib().or_rand(seed, stream, i)


def normal(seed, stream, i):
    return lib().or_normal(seed, stream, i)


def f32_to_f16(x):
    return lib().or_f32_to_f16(float(np.float32(x)))


def expf_survey(start_bits, end_bits, step=1):
    """(mismatches vs libm expf, mismatches vs double-rounded exp) over float bit patterns."""
    out = np.zeros(2, np.uint64)
    lib().or_expf_survey(start_bits, end_bits, step, out)
    return int(out[0]), int(out[1])


def ref_dequant_table():
    """Run oracle/_ref/ref_dequant (the reference's own decoders); None when not built."""
    if not os.path.exists(REF_DEQUANT):
        return None
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        out = os.path.join(d, "ref.bin")
        subprocess.run([REF_DEQUANT, out], check=True)
        data = np.fromfile(out, dtype="<f4")
    return data[:65536], data[65536:].reshape(256, 64)


# ------------------------------------------- fixture-model kernels (part 2)
# Restatements of the kernels StrataEngine.step uses outside the MoE stage
# (strata_oracle_model.c). Buffers the reference kernel updates in place
# (Residual, History, State, Keys/Values) are float32 arrays updated in place.
def logf(x):
    return np.float32(lib().or_logf(float(np.float32(x))))


def sinf(x):
    return np.float32(lib().or_sinf(float(np.float32(x))))


def cosf(x):
    return np.float32(lib().or_cosf(float(np.float32(x))))


def math_survey(fn, start_bits, end_bits, step=1):
    """fn 0 logf, 1 sinf, 2 cosf: (mismatches vs libm, mismatches beyond one ulp)."""
    out = np.zeros(2, np.uint64)
    lib().or_math_survey({"logf": 0, "sinf": 1, "cosf": 2}[fn], start_bits, end_bits, step, out)
    return int(out[0]), int(out[1])


def embedding(residual, width, streams, values=None, codes=None, scales=None, offsets=None, output_offset=0,
              fmt=0, bits=0, group_size=1, bias=0, codebook=0, has_offset=0):
    keep = [None if a is None else (f32(a) if a is not codes else u32(a)) for a in (values, codes, scales, offsets)]
    lib().or_embedding(*[_ptr(a) for a in keep], residual, width, streams, output_offset, fmt, bits, group_size,
                       bias, codebook, has_offset)
    return residual


def rope_frequencies(rotary, base):
    hi, lo = np.zeros(rotary // 2, np.float32), np.zeros(rotary // 2, np.float32)
    lib().or_rope_frequencies(hi, lo, rotary, float(np.float32(base)))
    return hi, lo


def rope_table(hi, lo, rotary, context):
    cos, sin = np.zeros(context * rotary // 2, np.float32), np.zeros(context * rotary // 2, np.float32)
    lib().or_rope_table(f32(hi), f32(lo), cos, sin, rotary, context)
    return cos, sin


def rope_position(X, cos, sin, dim, heads, rotary, position, tokens=1):
    Y = np.zeros(dim * heads * tokens, np.float32)
    lib().or_rope_position(f32(X), f32(cos), f32(sin), Y, dim, heads, rotary, position, tokens)
    return Y


def hc_mix(norm_, gate, width, streams):
    out = np.zeros(width, np.float32)
    lib().or_hc_mix(f32(norm_), f32(gate), out, width, streams)
    return out


def hc_write(residual, output, inject, width, streams):
    lib().or_hc_write(residual, f32(output), f32(inject), width, streams)
    return residual


def conv(history, X, W, channels, taps, dilation, activation=1):
    Y = np.zeros(channels, np.float32)
    lib().or_conv(history, f32(X), f32(W), Y, channels, taps, dilation, activation)
    return Y


def gdn_gates(alpha, beta, A, dt, heads):
    decay, strength = np.zeros(heads, np.float32), np.zeros(heads, np.float32)
    lib().or_gdn_gates(f32(alpha), f32(beta), f32(A), f32(dt), decay, strength, heads)
    return decay, strength


def gdn_step(state, q, k, v, decay, beta, dim, key_heads, value_heads):
    Y = np.zeros(dim * value_heads, np.float32)
    lib().or_gdn_step(state, f32(q), f32(k), f32(v), f32(decay), f32(beta), Y, dim, key_heads, value_heads)
    return Y


def slice_(X, width, rows=1, stride=None, offset=0):
    Y = np.zeros(width * rows, np.float32)
    lib().or_slice(f32(X), Y, width, rows, width if stride is None else stride, offset)
    return Y


def kv_append(k, v, keys, values, width, position):
    lib().or_kv_append(f32(k), f32(v), keys, values, width, position)


def attention(Q, keys, values, cells, dim, heads, kv_heads, count, scale):
    Y = np.zeros(dim * heads, np.float32)
    lib().or_attention(f32(Q), f32(keys), f32(values), i32(cells), Y, dim, heads, kv_heads, count,
                       float(np.float32(scale)))
    return Y


def attention_gate(attn, full_q, dim, heads):
    Y = np.zeros(dim * heads, np.float32)
    lib().or_attention_gate(f32(attn), f32(full_q), Y, dim, heads)
    return Y


def ple_gate(key, query, width, streams):
    gate = np.zeros(streams, np.float32)
    lib().or_ple_gate(f32(key), f32(query), gate, width, streams)
    return gate


def ple_broadcast(value, gate, width, streams):
    Y = np.zeros(width * streams, np.float32)
    lib().or_ple_broadcast(f32(value), f32(gate), Y, width, streams)
    return Y


def ple_add(residual, gated, conv_, n):
    lib().or_ple_add(residual, f32(gated), f32(conv_), n)
    return residual


def argmax(logits, count):
    return int(lib().or_argmax(f32(logits), count))


def bf16_project(X, codes, cols, rows, tokens, output_stride=None, output_offset=0, Y=None):
    output_stride = rows if output_stride is None else output_stride
    Y = np.zeros(tokens * output_stride, np.float32) if Y is None else Y
    lib().or_bf16_project(f32(X), u32(codes), Y, cols, rows, tokens, output_stride, output_offset)
    return Y


def quant_gemv(X, codes, scales, offsets, cols, rows, bits, group_size, bias, codebook, has_offset):
    """strata_quant_gemv (kernels/strata.cu:134-155): strata_quant_project's
    arithmetic for one token, Y[row]."""
    return quant_project(X, codes, scales, offsets, np.zeros(rows, np.float32), cols, rows, 1, rows, 0, bits,
                         group_size, bias, codebook, has_offset)


def ple_decode(packed_u32, count):
    out = np.zeros(count, np.float32)
    lib().or_ple_decode(u32(packed_u32), out, count)
    return out


def embed(row, width, streams):
    out = np.zeros(width * streams, np.float32)
    lib().or_embed(f32(row), out, width, streams)
    return out


def rope(X, cos, sin, dim, heads, rotary):
    Y = np.zeros(dim * heads, np.float32)
    lib().or_rope(f32(X), f32(cos), f32(sin), Y, dim, heads, rotary)
    return Y


# ------------------------------------------------ prompt (batch) kernels
def embed_batch(rows, width, streams, tokens):
    out = np.zeros(width * streams * tokens, np.float32)
    lib().or_embed_batch(f32(rows), out, width, streams, tokens)
    return out


def hc_mix_batch(norm_, gate, width, streams, tokens):
    out = np.zeros(width * tokens, np.float32)
    lib().or_hc_mix_batch(f32(norm_), f32(gate), out, width, streams, tokens)
    return out


def hc_write_batch(residual, output, inject, width, streams, tokens):
    lib().or_hc_write_batch(residual, f32(output), f32(inject), width, streams, tokens)
    return residual


def conv_batch(history, X, W, channels, taps, dilation, activation, tokens):
    Y = np.zeros(channels * tokens, np.float32)
    lib().or_conv_batch(history, f32(X), f32(W), Y, channels, taps, dilation, activation, tokens)
    return Y


def gdn_gates_batch(alpha, beta, A, dt, heads, tokens):
    decay, strength = np.zeros(heads * tokens, np.float32), np.zeros(heads * tokens, np.float32)
    lib().or_gdn_gates_batch(f32(alpha), f32(beta), f32(A), f32(dt), decay, strength, heads, tokens)
    return decay, strength


def gdn_batch(state, q, k, v, decay, beta, dim, key_heads, value_heads, tokens):
    Y = np.zeros(dim * value_heads * tokens, np.float32)
    lib().or_gdn_batch(state, f32(q), f32(k), f32(v), f32(decay), f32(beta), Y, dim, key_heads, value_heads, tokens)
    return Y


def rope_batch(X, cos, sin, dim, heads, rotary, tokens):
    Y = np.zeros(dim * heads * tokens, np.float32)
    lib().or_rope_batch(f32(X), f32(cos), f32(sin), Y, dim, heads, rotary, tokens)
    return Y


def kv_append_batch(k, v, keys, values, width, position, tokens):
    lib().or_kv_append_batch(f32(k), f32(v), keys, values, width, position, tokens)


def attention_gate_batch(attn, full_q, dim, heads, tokens):
    Y = np.zeros(dim * heads * tokens, np.float32)
    lib().or_attention_gate_batch(f32(attn), f32(full_q), Y, dim, heads, tokens)
    return Y


def ple_broadcast_batch(value, gate, width, streams, tokens):
    Y = np.zeros(width * streams * tokens, np.float32)
    lib().or_ple_broadcast_batch(f32(value), f32(gate), Y, width, streams, tokens)
    return Y


def attention_batch(Q, keys, values, dim, heads, kv_heads, position, scale, tokens):
    Y = np.zeros(dim * heads * tokens, np.float32)
    lib().or_attention_batch(f32(Q), f32(keys), f32(values), Y, dim, heads, kv_heads, position,
                             float(np.float32(scale)), tokens)
    return Y
