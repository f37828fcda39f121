"""ctypes binding of libgemma_hip.so (include/gemma_hip.h).

This mirrors the reference's GPU interface for Python callers (tests, bench):
  Context      <- GpuContext / GpuEngine (src/gpu/context.zig, src/gpu/kernels.zig)
  Buffer       <- GpuBuffer (src/gpu/buffer.zig)
  Model        <- GpuModelContext + gpuDispatchForwardToken
                  (src/gpu/model_gpu.zig, src/gpu/model_dispatch.zig)
Every call goes through the C ABI; a non-zero status raises GhError with the
library's message.  There is no fallback: without the built library or a
gfx950 device the calls fail.
"""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libgemma_hip.so")

QUANT_NONE, QUANT_Q8, QUANT_Q4 = 0, 1, 2

_vp = C.c_void_p
_sz = C.c_size_t
_u32 = C.c_uint32
_u64 = C.c_uint64
_f32 = C.c_float
_f64 = C.c_double
_i = C.c_int

# name -> (restype, argtypes); the single table of the ABI's signatures.
_SIGS = {
    "gh_device_count": (_i, []),
    "gh_context_init": (_i, [C.c_char_p, C.POINTER(_vp)]),
    "gh_context_deinit": (None, [_vp]),
    "gh_context_device_name": (C.c_char_p, [_vp]),
    "gh_last_error": (C.c_char_p, []),
    "gh_sync": (_i, [_vp]),
    "gh_buffer_alloc": (_i, [_vp, _sz, C.POINTER(_vp)]),
    "gh_buffer_free": (_i, [_vp, _vp]),
    "gh_buffer_write": (_i, [_vp, _vp, _vp, _sz]),
    "gh_buffer_read": (_i, [_vp, _vp, _vp, _sz]),
    "gh_buffer_copy": (_i, [_vp, _vp, _vp, _sz]),
    "gh_buffer_fill_u32": (_i, [_vp, _vp, _u32, _sz]),
    "gh_read_probe": (_i, [_vp, _vp, _sz, _u32, _u32, _u32, _vp]),
    "gh_event_create": (_i, [_vp, C.POINTER(_vp)]),
    "gh_event_record": (_i, [_vp, _vp]),
    "gh_event_elapsed_ms": (_i, [_vp, _vp, C.POINTER(_f32)]),
    "gh_event_destroy": (_i, [_vp]),
    "gh_graph_begin": (_i, [_vp]),
    "gh_graph_end": (_i, [_vp, C.POINTER(_vp)]),
    "gh_graph_launch": (_i, [_vp, _vp]),
    "gh_graph_destroy": (_i, [_vp]),
    "gh_quantized_row_words": (_sz, [_sz, _i]),
    "gh_quantized_size_bytes": (_sz, [_sz, _sz, _i]),
    "gh_quantize_matrix": (_i, [_vp, _vp, _sz, _sz, _i, _i]),
    "gh_quantize_matrix_dev": (_i, [_vp, _vp, _vp, _sz, _sz, _i]),
    "gh_synth_normal_f32": (_i, [_vp, _sz, _u64, _u64, _f64, _f64, _u64]),
    "gh_synth_normal_bf16": (_i, [_vp, _sz, _u64, _u64, _f64, _f64, _u64]),
    "gh_synth_normal_f32_dev": (_i, [_vp, _vp, _sz, _u64, _u64, _f64, _f64, _u64]),
    "gh_synth_normal_bf16_dev": (_i, [_vp, _vp, _sz, _u64, _u64, _f64, _f64, _u64]),
    "gh_synth_uniform_u32": (_i, [_vp, _sz, _u64, _u64, _u32]),
    "gh_gemv_q4": (_i, [_vp, _vp, _vp, _vp, _u32, _u32]),
    "gh_gemv_q8": (_i, [_vp, _vp, _vp, _vp, _u32, _u32]),
    "gh_gemv_bf16": (_i, [_vp, _vp, _vp, _vp, _u32, _u32]),
    "gh_gate_up_geglu_q4": (_i, [_vp, _vp, _vp, _vp, _vp, _u32, _u32]),
    "gh_rmsnorm": (_i, [_vp, _vp, _vp, _vp, _u32, _f32]),
    "gh_add_rmsnorm": (_i, [_vp, _vp, _vp, _vp, _vp, _u32, _f32, _f32]),
    "gh_qkv_rope": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32,
                         _u32, _f32, _f32]),
    "gh_decode_attn": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _f32, _u32]),
    "gh_argmax": (_i, [_vp, _vp, _vp, _u32]),
    "gh_qkv_rope_attn": (_i, [_vp] * 11 + [_u32] * 5 + [_f32, _f32, _u32, _vp]),
    "gh_qkv_rope_attn_noalloc": (_i, [_vp] * 11 + [_u32] * 5 + [_f32, _f32, _u32, _vp]),
    "gh_rope_table": (_i, [_vp, _vp, _u32, _f32, _vp]),
    "gh_prefill_gemm": (_i, [_vp, _i, _vp, _vp, _vp, _u32, _u32, _u32]),
    "gh_prefill_gate_up_geglu": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _u32, _u32, _u32]),
}

class XPrologue(C.Structure):
    """gh_xprologue: the x prologue of the fused GEMV entry points."""
    _fields_ = [("x", _vp), ("r", _vp), ("r_norm", _vp), ("norm", _vp), ("x_out", _vp),
                ("scalar", _f32), ("eps", _f32), ("mode", _u32)]


_SIGS.update({
    "gh_norm_gemv": (_i, [_vp, _i, _vp, _vp, _u32, _u32, C.POINTER(XPrologue)]),
    "gh_norm_gate_up_geglu": (_i, [_vp, _i, _vp, _vp, _vp, _u32, _u32, C.POINTER(XPrologue)]),
    "gh_norm_gemv_argmax_q8": (_i, [_vp, _vp, _vp, _vp, _u32, _u32, C.POINTER(XPrologue)]),
    "gh_norm_gemv_argmax_bf16": (_i, [_vp, _vp, _vp, _vp, _u32, _u32, C.POINTER(XPrologue)]),
})

class ModelConfig(C.Structure):
    """gh_model_config (ModelConfig, src/model/types.zig:43-61)."""
    _fields_ = [("vocab_size", _u32), ("hidden_size", _u32), ("intermediate_size", _u32),
                ("num_hidden_layers", _u32), ("num_attention_heads", _u32),
                ("num_key_value_heads", _u32), ("num_global_key_value_heads", _u32),
                ("head_dim", _u32), ("global_head_dim", _u32), ("attention_k_eq_v", _u32),
                ("max_slots", _u32), ("rms_norm_eps", _f32), ("rope_theta", _f32),
                ("rope_theta_full", _f32), ("layer_types", C.c_uint8 * 64)]


class LayerWeights(C.Structure):
    """gh_layer_weights (LayerWeights, src/model/types.zig:13-41)."""
    _fields_ = [(n, _vp) for n in ("input_layernorm", "q_proj", "k_proj", "v_proj", "o_proj",
                                   "q_norm", "k_norm", "post_attention_layernorm",
                                   "pre_feedforward_layernorm", "gate_proj", "up_proj",
                                   "down_proj", "post_feedforward_layernorm")] + \
        [("layer_scalar", _f32)]


_SIGS.update({
    "gh_ring_create": (_i, [_u32, _u32, _u32, _u32, C.POINTER(_vp)]),
    "gh_ring_destroy": (None, [_vp]),
    "gh_ring_total_slots": (_u32, [_vp]),
    "gh_ring_slot_index": (_u32, [_vp, _u64]),
    "gh_ring_activate_slot": (_u32, [_vp, _u32, _u64]),
    "gh_ring_clear_recall": (None, [_vp]),
    "gh_ring_activate_recall": (_u32, [_vp, _u32, _u32, _u64]),
    "gh_ring_active_slots": (_u32, [_vp, _u32, _u64, _vp, _u32]),
    "gh_model_init": (_i, [_vp, C.POINTER(ModelConfig), C.POINTER(LayerWeights), _vp, _vp, _i,
                           _f32, C.POINTER(_vp)]),
    "gh_model_init_synthetic": (_i, [_vp, C.POINTER(ModelConfig), _i, _u64, C.POINTER(_vp)]),
    "gh_model_deinit": (None, [_vp]),
    "gh_dispatch_forward_token": (_i, [_vp, _vp, _i, _u64, _u32, _vp, _u32, C.POINTER(_u32)]),
    "gh_model_prefill": (_i, [_vp, _vp, _u32, _vp, _vp, _vp, _u32, _vp, _i, C.POINTER(_u32)]),
    "gh_model_embed": (_i, [_vp, _u32, _vp]),
    "gh_model_ring_init": (_i, [_vp, _u32, _u32, _u32]),
    "gh_model_forward_clock": (_i, [_vp, _vp, _i, _u64, C.POINTER(_u32)]),
    "gh_model_ring_prefill": (_i, [_vp, _vp, _u32, _u64, _i, C.POINTER(_u32)]),
    "gh_model_ring_clear_recall": (_i, [_vp]),
    "gh_model_submit_prerecorded": (_i, [_vp, _i]),
    "gh_model_write_recall_kv": (_i, [_vp, _u32, _u32, _vp, _vp, _u64]),
    "gh_model_set_trace": (_i, [_vp, _i]),
    "gh_model_set_quiescence": (_i, [_vp, _f32]),
    "gh_model_tensor_bytes": (_sz, [_vp, _i, _i]),
    "gh_model_read_tensor": (_i, [_vp, _i, _i, _vp, _sz]),
    "gh_model_write_tensor": (_i, [_vp, _i, _i, _vp, _sz]),
})

# gh_tensor
(T_QKV, T_O_PROJ, T_GATE, T_UP, T_DOWN, T_INPUT_NORM, T_Q_NORM, T_K_NORM, T_POST_ATTN_NORM,
 T_PRE_FFN_NORM, T_POST_FFN_NORM, T_K_CACHE, T_V_CACHE) = range(13)
T_LM_HEAD, T_FINAL_NORM, T_EMBED, T_LOGITS, T_HIDDEN = 20, 21, 22, 23, 24
T_STEP, T_ACTIVE, T_RING_CLOCKS, T_RING_FLAGS, T_TRACE = 25, 26, 27, 28, 29
T_GATE_FLAGS, T_GATE_PREV, T_PREFILL_TRACE = 30, 31, 32
# gh_graph_kind
GRAPH_DECODE, GRAPH_PREFILL = 0, 1

_lib = None


class GhError(RuntimeError):
    pass


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise GhError("libgemma_hip.so is not built (run ai-research_amd/build.py)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def exported_symbols():
    return list(_SIGS)


def _check(st, what=""):
    if st != 0:
        msg = lib().gh_last_error().decode(errors="replace")
        raise GhError("%s failed (status %d): %s" % (what, st, msg))


def device_count():
    return lib().gh_device_count()


def _ptr(a):
    return a.ctypes.data_as(_vp)


# ---- host-side routines (no device needed) ---------------------------------
def quantize_matrix(w_bf16, mode, nthreads=0):
    """quantizeMatrix (src/quant.zig:92-162) on the host."""
    w = np.ascontiguousarray(w_bf16, np.uint16)
    rows, cols = w.shape
    out = np.zeros((rows, lib().gh_quantized_row_words(cols, mode)), np.uint32)
    _check(lib().gh_quantize_matrix(_ptr(out), _ptr(w), rows, cols, mode, nthreads),
           "gh_quantize_matrix")
    return out


def synth_normal(n, seed, stream, mean=0.0, std=1.0, bf16=False, offset=0):
    out = np.empty(n, np.uint16 if bf16 else np.float32)
    fn = lib().gh_synth_normal_bf16 if bf16 else lib().gh_synth_normal_f32
    _check(fn(_ptr(out), n, seed, stream, mean, std, offset), "gh_synth_normal")
    return out


def synth_uniform_u32(n, seed, stream, bound):
    out = np.empty(n, np.uint32)
    _check(lib().gh_synth_uniform_u32(_ptr(out), n, seed, stream, bound), "gh_synth_uniform_u32")
    return out


class Buffer:
    """A device allocation (GpuBuffer, src/gpu/buffer.zig:13-53)."""

    def __init__(self, ctx, nbytes):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = _vp()
        _check(lib().gh_buffer_alloc(ctx.h, self.nbytes, C.byref(p)), "gh_buffer_alloc")
        self.ptr = p.value

    def write(self, arr, offset=0):
        a = np.ascontiguousarray(arr)
        assert offset + a.nbytes <= self.nbytes
        _check(lib().gh_buffer_write(self.ctx.h, self.ptr + offset, _ptr(a), a.nbytes),
               "gh_buffer_write")
        return self

    def read(self, dtype, count=None, offset=0):
        dtype = np.dtype(dtype)
        n = (self.nbytes - offset) // dtype.itemsize if count is None else int(count)
        out = np.empty(n, dtype)
        _check(lib().gh_buffer_read(self.ctx.h, _ptr(out), self.ptr + offset, out.nbytes),
               "gh_buffer_read")
        return out

    def free(self):
        if self.ptr:
            _check(lib().gh_buffer_free(self.ctx.h, self.ptr), "gh_buffer_free")
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr and self.ctx.h:
                lib().gh_buffer_free(self.ctx.h, self.ptr)
        except Exception:
            pass


class Context:
    """GpuContext + GpuEngine: one gfx950 device, one in-order stream."""

    def __init__(self, code_object_dir=None):
        h = _vp()
        d = code_object_dir.encode() if code_object_dir else None
        _check(lib().gh_context_init(d, C.byref(h)), "gh_context_init")
        self.h = h.value

    @property
    def device_name(self):
        return lib().gh_context_device_name(self.h).decode()

    def close(self):
        if self.h:
            lib().gh_context_deinit(self.h)
            self.h = None

    def sync(self):
        _check(lib().gh_sync(self.h), "gh_sync")

    # ---- memory
    def alloc(self, nbytes):
        return Buffer(self, nbytes)

    def upload(self, arr):
        a = np.ascontiguousarray(arr)
        return Buffer(self, max(a.nbytes, 4)).write(a)

    def copy(self, dst, src, nbytes, dst_off=0, src_off=0):
        _check(lib().gh_buffer_copy(self.h, _addr(dst) + dst_off, _addr(src) + src_off, nbytes),
               "gh_buffer_copy")

    def fill_u32(self, buf, value, count):
        _check(lib().gh_buffer_fill_u32(self.h, _addr(buf), value, count), "gh_buffer_fill_u32")

    def read_probe(self, buf, nbytes, per_lane, contiguous, grid, sums):
        """HBM read-bandwidth probe: reads nbytes of buf once (gh_read_probe)."""
        _check(lib().gh_read_probe(self.h, _addr(buf), nbytes, per_lane, contiguous, grid,
                                   _addr(sums)), "gh_read_probe")

    # ---- events
    def event(self):
        e = _vp()
        _check(lib().gh_event_create(self.h, C.byref(e)), "gh_event_create")
        return e.value

    def record(self, ev):
        _check(lib().gh_event_record(self.h, ev), "gh_event_record")

    @staticmethod
    def elapsed_ms(a, b):
        ms = _f32()
        _check(lib().gh_event_elapsed_ms(a, b, C.byref(ms)), "gh_event_elapsed_ms")
        return ms.value

    @staticmethod
    def destroy_event(ev):
        lib().gh_event_destroy(ev)

    # ---- pre-recorded work (hipGraph capture of the context stream)
    def graph_begin(self):
        _check(lib().gh_graph_begin(self.h), "gh_graph_begin")

    def graph_end(self):
        g = _vp()
        _check(lib().gh_graph_end(self.h, C.byref(g)), "gh_graph_end")
        return g.value

    def graph_launch(self, g):
        _check(lib().gh_graph_launch(self.h, g), "gh_graph_launch")

    @staticmethod
    def graph_destroy(g):
        lib().gh_graph_destroy(g)

    # ---- quantization / synthetic data on the device
    def quantize_dev(self, dst, src_bf16, rows, cols, mode):
        _check(lib().gh_quantize_matrix_dev(self.h, _addr(dst), _addr(src_bf16), rows, cols, mode),
               "gh_quantize_matrix_dev")

    def synth_normal_dev(self, dst, n, seed, stream, mean=0.0, std=1.0, bf16=False, offset=0):
        fn = lib().gh_synth_normal_bf16_dev if bf16 else lib().gh_synth_normal_f32_dev
        _check(fn(self.h, _addr(dst), n, seed, stream, mean, std, offset), "gh_synth_normal_dev")

    # ---- engine kernels (GpuEngine.record*)
    def gemv_q4(self, W, X, Y, M, K):
        _check(lib().gh_gemv_q4(self.h, _addr(W), _addr(X), _addr(Y), M, K), "gh_gemv_q4")

    def gemv_q8(self, W, X, Y, M, K):
        _check(lib().gh_gemv_q8(self.h, _addr(W), _addr(X), _addr(Y), M, K), "gh_gemv_q8")

    def gemv_bf16(self, W, X, Y, M, K):
        _check(lib().gh_gemv_bf16(self.h, _addr(W), _addr(X), _addr(Y), M, K), "gh_gemv_bf16")

    def gate_up_geglu_q4(self, Wg, Wu, X, Y, M, K):
        _check(lib().gh_gate_up_geglu_q4(self.h, _addr(Wg), _addr(Wu), _addr(X), _addr(Y), M, K),
               "gh_gate_up_geglu_q4")

    @staticmethod
    def prologue(x, mode=0, norm=None, r=None, r_norm=None, x_out=None, scalar=1.0, eps=1e-6):
        a = lambda b: _addr(b) if b is not None else None  # noqa: E731
        return XPrologue(a(x), a(r), a(r_norm), a(norm), a(x_out), scalar, eps, mode)

    def norm_gemv(self, quant, W, Y, M, K, pro):
        _check(lib().gh_norm_gemv(self.h, quant, _addr(W), _addr(Y), M, K, C.byref(pro)),
               "gh_norm_gemv")

    def norm_gate_up_geglu(self, quant, Wg, Wu, Y, M, K, pro):
        _check(lib().gh_norm_gate_up_geglu(self.h, quant, _addr(Wg), _addr(Wu), _addr(Y), M, K,
                                           C.byref(pro)), "gh_norm_gate_up_geglu")

    def norm_gemv_argmax_q8(self, W, logits, token, M, K, pro):
        _check(lib().gh_norm_gemv_argmax_q8(self.h, _addr(W), _addr(logits) if logits else None,
                                            _addr(token), M, K, C.byref(pro)),
               "gh_norm_gemv_argmax_q8")

    def norm_gemv_argmax_bf16(self, W, logits, token, M, K, pro):
        _check(lib().gh_norm_gemv_argmax_bf16(self.h, _addr(W), _addr(logits) if logits else None,
                                              _addr(token), M, K, C.byref(pro)),
               "gh_norm_gemv_argmax_bf16")

    def rmsnorm(self, X, W, Y, dim, eps=1e-6):
        _check(lib().gh_rmsnorm(self.h, _addr(X), _addr(W), _addr(Y), dim, eps), "gh_rmsnorm")

    def add_rmsnorm(self, X, R, W, Y, dim, eps=1e-6, scalar=1.0):
        _check(lib().gh_add_rmsnorm(self.h, _addr(X), _addr(R), _addr(W), _addr(Y), dim, eps,
                                    scalar), "gh_add_rmsnorm")

    def qkv_rope(self, Q_in, K_in, V_in, Qn, Kn, Q_out, K_cache, V_cache, step, num_q, num_kv,
                 head_dim, rotary_dim, k_eq_v, theta, eps=1e-6):
        _check(lib().gh_qkv_rope(self.h, _addr(Q_in), _addr(K_in), _addr(V_in) if V_in else None,
                                 _addr(Qn), _addr(Kn), _addr(Q_out), _addr(K_cache),
                                 _addr(V_cache), _addr(step), num_q, num_kv, head_dim, rotary_dim,
                                 int(k_eq_v), theta, eps), "gh_qkv_rope")

    def decode_attn(self, Q, K_cache, V_cache, active, out, step, head_dim, kv_dim, gqa_ratio,
                    num_q_heads, inv_sqrt_dim=1.0):
        _check(lib().gh_decode_attn(self.h, _addr(Q), _addr(K_cache), _addr(V_cache),
                                    _addr(active), _addr(out), _addr(step), head_dim, kv_dim,
                                    gqa_ratio, inv_sqrt_dim, num_q_heads), "gh_decode_attn")

    def qkv_rope_attn(self, Q, K, V, Qn, Kn, K_cache, V_cache, active, step, out, num_q, num_kv,
                      head_dim, rot, k_eq_v, theta, eps=1e-6, max_slots=640, table=None):
        _check(lib().gh_qkv_rope_attn(self.h, _addr(Q), _addr(K), _addr(V), _addr(Qn), _addr(Kn),
                                      _addr(K_cache), _addr(V_cache), _addr(active), _addr(step),
                                      _addr(out), num_q, num_kv, head_dim, rot, int(k_eq_v),
                                      theta, eps, max_slots,
                                      None if table is None else _addr(table)),
               "gh_qkv_rope_attn")

    def qkv_rope_attn_noalloc(self, Q, K, V, Qn, Kn, K_cache, V_cache, active, step, out, num_q,
                              num_kv, head_dim, rot, k_eq_v, theta, eps=1e-6, max_slots=640,
                              table=None):
        _check(lib().gh_qkv_rope_attn_noalloc(self.h, _addr(Q), _addr(K), _addr(V), _addr(Qn),
                                              _addr(Kn), _addr(K_cache), _addr(V_cache),
                                              _addr(active), _addr(step), _addr(out), num_q,
                                              num_kv, head_dim, rot, int(k_eq_v), theta, eps,
                                              max_slots, None if table is None else _addr(table)),
               "gh_qkv_rope_attn_noalloc")

    def rope_table(self, step, rot, theta, table):
        _check(lib().gh_rope_table(self.h, _addr(step), rot, theta, _addr(table)), "gh_rope_table")

    def argmax(self, logits, out_token, vocab):
        _check(lib().gh_argmax(self.h, _addr(logits), _addr(out_token), vocab), "gh_argmax")

    def prefill_gemm(self, mode, W, A, C, T, N, K):
        """C [T][N] = A [T][K] . deq(W)^T on the matrix cores (A, C f32)."""
        _check(lib().gh_prefill_gemm(self.h, mode, _addr(W), _addr(A), _addr(C), T, N, K),
               "gh_prefill_gemm")

    def prefill_gate_up_geglu(self, mode, Wg, Wu, A, act, T, N, K):
        _check(lib().gh_prefill_gate_up_geglu(self.h, mode, _addr(Wg), _addr(Wu), _addr(A),
                                              _addr(act), T, N, K), "gh_prefill_gate_up_geglu")


def _addr(b):
    if isinstance(b, Buffer):
        return b.ptr
    return int(b)


class Ring:
    """DynamicRingBuffer slot bookkeeping (src/ring_buffer.zig:7-147)."""

    def __init__(self, num_layers, num_anchors, window_size, num_recall):
        h = _vp()
        _check(lib().gh_ring_create(num_layers, num_anchors, window_size, num_recall,
                                    C.byref(h)), "gh_ring_create")
        self.h = h.value
        self.total_slots = lib().gh_ring_total_slots(self.h)

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.gh_ring_destroy(self.h)
            self.h = None

    def slot_index(self, clock):
        return lib().gh_ring_slot_index(self.h, clock)

    def activate_slot(self, layer, clock):
        return lib().gh_ring_activate_slot(self.h, layer, clock)

    def clear_recall(self):
        lib().gh_ring_clear_recall(self.h)

    def activate_recall(self, layer, rank, clock):
        return lib().gh_ring_activate_recall(self.h, layer, rank, clock)

    def active_slots(self, layer, clock):
        out = np.zeros(self.total_slots, np.uint32)
        n = lib().gh_ring_active_slots(self.h, layer, clock, _ptr(out), self.total_slots)
        return out[:n].copy()


def model_config(vocab, hidden, intermediate, layers, heads, kv_heads, head_dim, max_slots,
                 global_kv_heads=None, global_head_dim=None, k_eq_v=False, eps=1e-6,
                 theta=10000.0, theta_full=1e6, full_layers=()):
    c = ModelConfig()
    c.vocab_size, c.hidden_size, c.intermediate_size = vocab, hidden, intermediate
    c.num_hidden_layers, c.num_attention_heads, c.num_key_value_heads = layers, heads, kv_heads
    c.num_global_key_value_heads = kv_heads if global_kv_heads is None else global_kv_heads
    c.head_dim = head_dim
    c.global_head_dim = head_dim if global_head_dim is None else global_head_dim
    c.attention_k_eq_v = int(k_eq_v)
    c.max_slots = max_slots
    c.rms_norm_eps, c.rope_theta, c.rope_theta_full = eps, theta, theta_full
    for l in full_layers:
        c.layer_types[l] = 1
    return c


class Model:
    """GpuModelContext: weights, K/V ring caches and the recorded graphs."""

    def __init__(self, ctx, cfg, mode=QUANT_Q4, seed=None, layers=None, embed=None,
                 final_norm=None):
        self.ctx, self.cfg = ctx, cfg
        h = _vp()
        if seed is not None:
            _check(lib().gh_model_init_synthetic(ctx.h, C.byref(cfg), mode, seed, C.byref(h)),
                   "gh_model_init_synthetic")
        else:
            self._keep = []
            arr = (LayerWeights * cfg.num_hidden_layers)()
            for i, d in enumerate(layers):
                for name, _ in LayerWeights._fields_[:-1]:
                    a = d.get(name)
                    if a is None:
                        setattr(arr[i], name, None)
                    else:
                        a = np.ascontiguousarray(a, np.uint16)
                        self._keep.append(a)
                        setattr(arr[i], name, a.ctypes.data)
                arr[i].layer_scalar = float(d.get("layer_scalar", 1.0))
            e = np.ascontiguousarray(embed, np.uint16)
            fn = None if final_norm is None else np.ascontiguousarray(final_norm, np.uint16)
            self._keep += [e, fn]
            _check(lib().gh_model_init(ctx.h, C.byref(cfg), arr, _ptr(e),
                                       _ptr(fn) if fn is not None else None, mode, 0.0,
                                       C.byref(h)), "gh_model_init")
        self.h = h.value

    def close(self):
        if self.h:
            lib().gh_model_deinit(self.h)
            self.h = None

    def forward(self, x, clock, slot_idx, active, want_logits=True):
        x = np.ascontiguousarray(x, np.float32)
        act = np.ascontiguousarray(active, np.uint32)
        tok = _u32()
        _check(lib().gh_dispatch_forward_token(self.h, _ptr(x), int(want_logits), clock, slot_idx,
                                               _ptr(act), act.size, C.byref(tok)),
               "gh_dispatch_forward_token")
        return tok.value

    def prefill(self, x, clocks, slots, actives, want_logits=True):
        """T tokens in one call; actives[t] is token t's active slot list."""
        x = np.ascontiguousarray(x, np.float32)
        T = x.shape[0]
        clocks = np.ascontiguousarray(clocks, np.uint64)
        slots = np.ascontiguousarray(slots, np.uint32)
        n_act = np.array([len(a) for a in actives], np.uint32)
        stride = int(n_act.max())
        act = np.zeros((T, stride), np.uint32)
        for t, a in enumerate(actives):
            act[t, :len(a)] = a
        tok = _u32()
        _check(lib().gh_model_prefill(self.h, _ptr(x), T, _ptr(clocks), _ptr(slots), _ptr(act),
                                      stride, _ptr(n_act), int(want_logits), C.byref(tok)),
               "gh_model_prefill")
        return tok.value

    # ---- device-resident ring (gh_model_ring_*) ----
    def ring_init(self, anchors, window, recall):
        _check(lib().gh_model_ring_init(self.h, anchors, window, recall), "gh_model_ring_init")

    def forward_clock(self, x, clock, want_logits=True):
        x = np.ascontiguousarray(x, np.float32)
        tok = _u32()
        _check(lib().gh_model_forward_clock(self.h, _ptr(x), int(want_logits), clock, C.byref(tok)),
               "gh_model_forward_clock")
        return tok.value

    def ring_prefill(self, x, first_clock, want_logits=True):
        x = np.ascontiguousarray(x, np.float32)
        tok = _u32()
        _check(lib().gh_model_ring_prefill(self.h, _ptr(x), x.shape[0], first_clock,
                                           int(want_logits), C.byref(tok)), "gh_model_ring_prefill")
        return tok.value

    def submit_prerecorded(self, which=0):
        """Replays the decode (0) or prefill (1) graph on the inputs the
        device holds (src/model/bench.zig:12-15's submitPreRecorded)."""
        _check(lib().gh_model_submit_prerecorded(self.h, which), "gh_model_submit_prerecorded")

    def ring_clear_recall(self):
        _check(lib().gh_model_ring_clear_recall(self.h), "gh_model_ring_clear_recall")

    def write_recall_kv(self, layer, rank, k, v, clock):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        _check(lib().gh_model_write_recall_kv(self.h, layer, rank, _ptr(k), _ptr(v), clock),
               "gh_model_write_recall_kv")

    def set_quiescence(self, threshold):
        _check(lib().gh_model_set_quiescence(self.h, threshold), "gh_model_set_quiescence")

    def set_trace(self, enable):
        _check(lib().gh_model_set_trace(self.h, int(enable)), "gh_model_set_trace")

    def embed(self, token):
        x = np.empty(self.cfg.hidden_size, np.float32)
        _check(lib().gh_model_embed(self.h, token, _ptr(x)), "gh_model_embed")
        return x

    def tensor_bytes(self, layer, t):
        return lib().gh_model_tensor_bytes(self.h, layer, t)

    def read(self, layer, t, dtype):
        n = self.tensor_bytes(layer, t)
        if n == 0:
            return None
        out = np.empty(n // np.dtype(dtype).itemsize, dtype)
        _check(lib().gh_model_read_tensor(self.h, layer, t, _ptr(out), out.nbytes),
               "gh_model_read_tensor")
        return out

    def write(self, layer, t, arr):
        a = np.ascontiguousarray(arr)
        _check(lib().gh_model_write_tensor(self.h, layer, t, _ptr(a), a.nbytes),
               "gh_model_write_tensor")
