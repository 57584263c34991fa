"""MI355X (gfx950) mixture-of-experts library: Python binding of libstrata_mi355x.so.

``Backend`` mirrors the reference's backend contract (src/backend.js:58-152):
``alloc(data_or_length, type)`` returns a buffer handle whose ``length`` is in
4-byte words, ``write / read / copy / zero / run(name, args, groups) / free /
idle / info / dispose``; ``run`` takes the reference's named arguments
(buffers and numbers) and workgroup counts of 64 lanes. The MoE layer entry
points (``moe_layer``, ``moe_route``, ``moe_dispatch``) run the whole stage on
the device. There is no CPU fallback: without the built library or a GPU the
constructor raises.
"""
import ctypes
import json
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libstrata_mi355x.so")

SM_OK = 0
ERRORS = {-1: "hip", -2: "argument", -3: "bounds", -4: "handle", -5: "no kernel", -6: "route", -7: "memory",
          -8: "fused decode fault"}
SM_E_FAULT = -8

_TYPES = {"f32": np.float32, "i32": np.int32, "u32": np.uint32}
_lib = None


class StrataError(RuntimeError):
    def __init__(self, code, message):
        super().__init__("%s (%s error %d)" % (message, ERRORS.get(code, "unknown"), code))
        self.code = code


class ArgumentError(StrataError, ValueError):
    """Invalid argument, the reference's RangeError (src/backend.js:6-14)."""


def lib():
    """Load libstrata_mi355x.so; raises when it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("libstrata_mi355x.so is not built; run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        u64, i, vp = ctypes.c_uint64, ctypes.c_int, ctypes.c_void_p
        pu64 = ctypes.POINTER(ctypes.c_uint64)
        sig = {
            "sm_init": (i, [i, ctypes.POINTER(vp)]),
            "sm_shutdown": (None, [vp]),
            "sm_last_error": (ctypes.c_char_p, [vp]),
            "sm_info": (i, [vp, ctypes.c_char_p, ctypes.c_size_t]),
            "sm_alloc": (i, [vp, u64, i, pu64]),
            "sm_free": (i, [vp, u64]),
            "sm_size": (i, [vp, u64, pu64]),
            "sm_write": (i, [vp, u64, u64, vp, u64]),
            "sm_read": (i, [vp, u64, u64, vp, u64]),
            "sm_copy": (i, [vp, u64, u64, u64, u64, u64]),
            "sm_zero": (i, [vp, u64, u64, u64]),
            "sm_sync": (i, [vp]),
            "sm_run": (i, [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32), pu64, i]),
            "sm_kernel_count": (i, []),
            "sm_kernel_name": (ctypes.c_char_p, [i]),
            "sm_kernel_signature": (ctypes.c_char_p, [ctypes.c_char_p]),
            "sm_moe_route": (i, [vp, u64, i, i, u64, u64, i, i, u64, u64, u64]),
            "sm_moe_dispatch": (i, [vp, u64, i, i, i, u64, u64, u64, u64, u64, u64]),
            "sm_moe_layer_workspace": (i, [i, i, i, i, i, pu64]),
            "sm_moe_layer": (i, [vp, u64, i, u64, u64, u64, u64, u64, u64, i, i, i, i, u64, u64, u64, u64, u64]),
            "sm_moe_layer_static": (i, [vp, u64, i, u64, u64, u64, u64, u64, u64, i, i, i, i, u64, u64, u64]),
            "sm_moe_block_workspace": (i, [i, i, i, i, i, pu64]),
            "sm_moe_block": (i, [vp, u64, i, u64, ctypes.c_float, u64, u64, u64, u64, u64, u64, i, i, i, i, u64, u64,
                                 u64, u64, u64]),
            "sm_stage_timing": (i, [vp, i]),
            "sm_stage_report": (i, [vp, ctypes.POINTER(ctypes.c_double), pu64, i]),
            "sm_stage_select": (i, [vp, ctypes.c_uint32]),
            "sm_graph_begin": (i, [vp]),
            "sm_graph_end": (i, [vp, ctypes.POINTER(i)]),
            "sm_graph_launch": (i, [vp, i]),
            "sm_graph_free": (i, [vp, i]),
            "sm_event_record": (i, [vp, i]),
            "sm_event_elapsed": (i, [vp, i, i, ctypes.POINTER(ctypes.c_float)]),
            "sm_synth_normal": (i, [vp, u64, u64, u64, u64, u64, ctypes.c_double]),
            "sm_synth_uniform_pm": (i, [vp, u64, u64, u64, u64, u64, ctypes.c_double]),
            "sm_synth_blobs": (i, [vp, u64, u64, u64, i, i, i, u64, u64, ctypes.c_double]),
            "sm_load_experts": (i, [vp, ctypes.c_char_p, u64, u64, i, u64, u64, u64, u64]),
            "sm_fused_fits": (i, [i, i]),
            "sm_moe_route_stats": (i, [vp, u64, i, i, i, i, i, pu64, ctypes.POINTER(i)]),
            "sm_fused_reset": (i, [vp]),
            "sm_fused_test_hooks": (i, [vp, ctypes.c_uint32, i]),
            "sm_prefetch_router": (i, [vp, ctypes.c_uint64, i, i]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def kernel_signatures():
    """{name: [(param, type), ...]} in the reference's parameter order."""
    L = lib()
    out = {}
    for k in range(L.sm_kernel_count()):
        name = L.sm_kernel_name(k).decode()
        sig = L.sm_kernel_signature(name.encode()).decode()
        out[name] = [tuple(p.split(":")) for p in sig.split(",")]
    return out


def blob_layout(width, ff):
    """Byte offsets of one Q2 expert blob (vendor/strata/tools/pack_layer.py:54-65)."""
    gu = 0
    dn = 2 * ff * width // 4
    gus = dn + width * ff // 4
    ds = gus + 2 * ff * (width // 64) * 2
    end = ds + width * (ff // 64) * 2
    return {"gate_up_codes": gu, "down_codes": dn, "gate_up_scales": gus, "down_scales": ds, "blob_bytes": end}


class Buffer:
    __slots__ = ("handle", "nbytes", "type", "length")

    def __init__(self, handle, nbytes, type_):
        self.handle = handle
        self.nbytes = nbytes
        self.type = type_
        self.length = nbytes // 4

    def __repr__(self):
        return "Buffer(0x%x, %d bytes, %s)" % (self.handle, self.nbytes, self.type)


class Backend:
    """One HIP context on one GPU (kind 'hip')."""

    kind = "hip"

    def __init__(self, device=0):
        L = lib()
        ctx = ctypes.c_void_p()
        rc = L.sm_init(device, ctypes.byref(ctx))
        if rc != SM_OK:
            raise StrataError(rc, "sm_init failed: no usable HIP device %d" % device)
        self._ctx = ctx
        self.buffers = set()
        self._sigs = None

    # -------------------------------------------------------------- errors
    def _check(self, rc):
        if rc != SM_OK:
            msg = lib().sm_last_error(self._ctx).decode(errors="replace")
            raise (ArgumentError if rc in (-2, -3) else StrataError)(rc, msg)

    # ------------------------------------------------------------- buffers
    def alloc(self, data_or_length, type="f32", zero=True):
        """Length in 4-byte words, or an array uploaded as-is (src/backend.js:84-92)."""
        if type not in _TYPES:
            raise ValueError("Unsupported buffer type " + str(type))
        if isinstance(data_or_length, (int, np.integer)):
            n = int(data_or_length)
            if n < 1:
                raise ArgumentError(-2, "allocation must be an integer in [1, 2147483647]")
            nbytes, data = n * 4, None
        else:
            data = np.ascontiguousarray(data_or_length)
            nbytes = data.nbytes
        h = ctypes.c_uint64()
        self._check(lib().sm_alloc(self._ctx, nbytes, 1 if (zero and data is None) else 0, ctypes.byref(h)))
        buf = Buffer(h.value, nbytes, type)
        self.buffers.add(buf)
        if data is not None:
            self.write(buf, data)
        return buf

    def alloc_bytes(self, nbytes, zero=False):
        h = ctypes.c_uint64()
        self._check(lib().sm_alloc(self._ctx, nbytes, 1 if zero else 0, ctypes.byref(h)))
        buf = Buffer(h.value, nbytes, "u32")
        self.buffers.add(buf)
        return buf

    def write(self, buf, data, offset=0):
        """offset in 4-byte words (src/backend.js:93)."""
        data = np.ascontiguousarray(data)
        self._check(lib().sm_write(self._ctx, buf.handle, offset * 4, data.ctypes.data, data.nbytes))

    def write_bytes(self, buf, data, offset_bytes=0):
        data = np.ascontiguousarray(data)
        self._check(lib().sm_write(self._ctx, buf.handle, offset_bytes, data.ctypes.data, data.nbytes))

    def read(self, buf, type=None, count=None, offset=0):
        dt = _TYPES[type or buf.type]
        n = buf.length - offset if count is None else count
        out = np.empty(n, dt)
        self._check(lib().sm_read(self._ctx, buf.handle, offset * 4, out.ctypes.data, n * 4))
        return out

    def read_bytes(self, buf, nbytes=None, offset_bytes=0):
        n = buf.nbytes - offset_bytes if nbytes is None else nbytes
        out = np.empty(n, np.uint8)
        self._check(lib().sm_read(self._ctx, buf.handle, offset_bytes, out.ctypes.data, n))
        return out

    def copy(self, source, destination, count=None, source_offset=0, destination_offset=0):
        count = source.length if count is None else count
        self._check(lib().sm_copy(self._ctx, source.handle, source_offset * 4, destination.handle,
                                  destination_offset * 4, count * 4))

    def zero(self, buf):
        self._check(lib().sm_zero(self._ctx, buf.handle, 0, buf.nbytes))

    def free(self, buf):
        if buf not in self.buffers:
            return
        self.buffers.discard(buf)
        self._check(lib().sm_free(self._ctx, buf.handle))

    def idle(self):
        self._check(lib().sm_sync(self._ctx))

    def route_stats(self, workspace, tokens, width, ff, experts, topk):
        """(candidates, fallbacks) of the certified batch router's last call on
        this workspace, or None when the batch did not use it."""
        c, f = ctypes.c_uint64(0), ctypes.c_int(0)
        n = lib().sm_moe_route_stats(self._ctx, workspace.handle, tokens, width, ff, experts, topk, ctypes.byref(c),
                                     ctypes.byref(f))
        if n < 0:
            self._check(n)
        return (int(c.value), int(f.value)) if n > 0 else None

    def fused_reset(self):
        """Clears the single-launch decode layer's fault (sm_fused_reset)."""
        self._check(lib().sm_fused_reset(self._ctx))

    def prefetch_router(self, Wr, rows=0, width=0):
        """The router matrix of the layer after the next one, pulled into L2
        by the next single-launch decode layer (sm_prefetch_router); None
        clears the hint."""
        self._check(lib().sm_prefetch_router(self._ctx, Wr.handle if Wr is not None else 0, rows, width))

    def fused_test_hooks(self, spin_limit=0, withhold=False):
        """Test hook of the give-up path: poll limit (0 = default) and a collector
        that waits for a flag no block writes (sm_fused_test_hooks)."""
        self._check(lib().sm_fused_test_hooks(self._ctx, spin_limit, 1 if withhold else 0))

    sync = idle

    def info(self):
        b = ctypes.create_string_buffer(1024)
        n = lib().sm_info(self._ctx, b, 1024)
        if n < 0:
            self._check(n)
        return json.loads(b.value.decode())

    def dispose(self):
        if self._ctx:
            lib().sm_shutdown(self._ctx)
            self._ctx = None
            self.buffers.clear()

    def __del__(self):
        try:
            self.dispose()
        except Exception:
            pass

    # ------------------------------------------------------ kernels by name
    def run(self, name, args, groups):
        """backend.run(name, args, groups) with named arguments (src/backend.js:101-113)."""
        if self._sigs is None:
            self._sigs = kernel_signatures()
        sig = self._sigs.get(name)
        if sig is None:
            raise StrataError(-5, "Unknown kernel " + str(name))
        slots = (ctypes.c_uint64 * len(sig))()
        for k, (pname, ptype) in enumerate(sig):
            if pname not in args:
                raise ArgumentError(-2, "Missing %s.%s" % (name, pname))
            v = args[pname]
            if ptype.endswith("*"):
                if not isinstance(v, Buffer):
                    raise ArgumentError(-2, "%s.%s must be a buffer" % (name, pname))
                slots[k] = v.handle
            elif ptype == "f32":
                slots[k] = struct.unpack("<I", struct.pack("<f", float(v)))[0]
            else:
                iv = int(v)
                if iv != v:
                    raise ArgumentError(-2, "%s.%s must be an integer" % (name, pname))
                slots[k] = iv & 0xffffffff
        g = (ctypes.c_uint32 * 3)(*[int(x) for x in groups])
        self._check(lib().sm_run(self._ctx, name.encode(), g, slots, len(sig)))

    # -------------------------------------------------------------- MoE
    @staticmethod
    def moe_workspace_bytes(tokens, width, ff, experts, topk):
        n = ctypes.c_uint64()
        rc = lib().sm_moe_layer_workspace(tokens, width, ff, experts, topk, ctypes.byref(n))
        if rc != SM_OK:
            raise ArgumentError(rc, "invalid MoE geometry")
        return n.value

    def moe_route(self, X, tokens, width, Wr, experts, topk, ids, weights, logits=None, bias=None):
        self._check(lib().sm_moe_route(self._ctx, X.handle, tokens, width, Wr.handle, bias.handle if bias else 0,
                                       experts, topk, logits.handle if logits else 0, ids.handle, weights.handle))

    def moe_dispatch(self, ids, tokens, topk, experts, offsets, rows, parts, where, workspace):
        self._check(lib().sm_moe_dispatch(self._ctx, ids.handle, tokens, topk, experts, offsets.handle, rows.handle,
                                          parts.handle, where.handle, workspace.handle, workspace.nbytes))

    def moe_layer(self, X, tokens, Wr, arena, blob_stride, shared_blob, Wsg, width, ff, experts, topk, Y, ids,
                  weights, workspace, bias=None):
        self._check(lib().sm_moe_layer(self._ctx, X.handle, tokens, Wr.handle, bias.handle if bias else 0,
                                       arena.handle, blob_stride, shared_blob.handle, Wsg.handle, width, ff, experts,
                                       topk, Y.handle, ids.handle, weights.handle, workspace.handle,
                                       workspace.nbytes))

    def moe_layer_static(self, X, tokens, Wr, arena, blob_stride, shared_blob, Wsg, width, ff, experts, topk, Y, ids,
                         weights, bias=None):
        """sm_moe_layer without a workspace: the decode path on the library's
        static device scratch (at most 16 tokens; nothing is allocated)."""
        self._check(lib().sm_moe_layer_static(self._ctx, X.handle, tokens, Wr.handle, bias.handle if bias else 0,
                                              arena.handle, blob_stride, shared_blob.handle, Wsg.handle, width, ff,
                                              experts, topk, Y.handle, ids.handle, weights.handle))

    @staticmethod
    def moe_block_workspace_bytes(tokens, width, ff, experts, topk):
        n = ctypes.c_uint64()
        rc = lib().sm_moe_block_workspace(tokens, width, ff, experts, topk, ctypes.byref(n))
        if rc != SM_OK:
            raise ArgumentError(rc, "invalid MoE geometry")
        return n.value

    def moe_block(self, H, tokens, gamma, eps, Wr, arena, blob_stride, shared_blob, Wsg, width, ff, experts, topk,
                  Hout, ids, weights, workspace, bias=None):
        """Hout = H + MoE(RMSNorm(H; gamma, eps)), one layer of the stack."""
        self._check(lib().sm_moe_block(self._ctx, H.handle, tokens, gamma.handle, eps, Wr.handle,
                                       bias.handle if bias else 0, arena.handle, blob_stride, shared_blob.handle,
                                       Wsg.handle, width, ff, experts, topk, Hout.handle, ids.handle, weights.handle,
                                       workspace.handle, workspace.nbytes))

    # ------------------------------------------------------------ timing
    STAGES = ["decode_route", "decode_gate_up", "decode_down_combine", "prefill_route", "prefill_dispatch",
              "prefill_gate_up_gemm", "prefill_down_gemm", "prefill_combine", "decode_fused"]

    def stage_timing(self, enable=True):
        self._check(lib().sm_stage_timing(self._ctx, 1 if enable else 0))

    def stage_report(self):
        """{stage: (total_ms, calls)} accumulated since stage_timing(True)."""
        ms = (ctypes.c_double * 16)()
        calls = (ctypes.c_uint64 * 16)()
        n = lib().sm_stage_report(self._ctx, ms, calls, 16)
        if n < 0:
            self._check(n)
        return {self.STAGES[k]: (ms[k], calls[k]) for k in range(n)}

    def stage_select(self, mask=0xffffffff):
        self._check(lib().sm_stage_select(self._ctx, mask))

    def graph_begin(self):
        self._check(lib().sm_graph_begin(self._ctx))

    def graph_end(self):
        gid = ctypes.c_int()
        self._check(lib().sm_graph_end(self._ctx, ctypes.byref(gid)))
        return gid.value

    def graph_launch(self, gid):
        self._check(lib().sm_graph_launch(self._ctx, gid))

    def graph_free(self, gid):
        self._check(lib().sm_graph_free(self._ctx, gid))

    def event_record(self, slot):
        self._check(lib().sm_event_record(self._ctx, slot))

    def event_elapsed_ms(self, a, b):
        ms = ctypes.c_float()
        self._check(lib().sm_event_elapsed(self._ctx, a, b, ctypes.byref(ms)))
        return ms.value

    # --------------------------------------------------- synthetic inputs
    def synth_normal(self, buf, n, seed, stream, sigma, offset_bytes=0):
        self._check(lib().sm_synth_normal(self._ctx, buf.handle, offset_bytes, n, seed, stream, sigma))

    def synth_uniform_pm(self, buf, n, seed, stream, amp, offset_bytes=0):
        self._check(lib().sm_synth_uniform_pm(self._ctx, buf.handle, offset_bytes, n, seed, stream, amp))

    def load_experts(self, path, file_offset, blob_bytes, count, arena, stride, scales_offset, dst_offset=0):
        """Stream `count` blobs (back to back at file_offset of a pack's
        experts.bin) into `arena` at `stride`, then check their fp16 scales
        (PackStore.readExpertBlob, src/model.js:160-167)."""
        self._check(lib().sm_load_experts(self._ctx, os.fsencode(path), file_offset, blob_bytes, count,
                                          arena.handle, dst_offset, stride, scales_offset))

    def synth_blobs(self, buf, count, width, ff, seed, first_stream, sigma=0.05, stride=None, offset_bytes=0):
        stride = blob_layout(width, ff)["blob_bytes"] if stride is None else stride
        self._check(lib().sm_synth_blobs(self._ctx, buf.handle, offset_bytes, stride, count, width, ff, seed,
                                         first_stream, sigma))
