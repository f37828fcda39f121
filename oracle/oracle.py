"""ctypes binding of the CPU oracle (oracle/liboracle.so) -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker.  The product (ai-research_amd/) never
imports it.  Each wrapper names the reference function it restates; the
citations live in oracle.c.
"""
import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

QUANT_NONE, QUANT_Q8, QUANT_Q4 = 0, 1, 2

_u16p = C.POINTER(C.c_uint16)
_u32p = C.POINTER(C.c_uint32)
_f32p = C.POINTER(C.c_float)
_sz = C.c_size_t


def build():
    """Compile liboracle.so with its Makefile (gcc only)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        L.orc_bf16_from_f32.restype = C.c_uint16
        L.orc_bf16_from_f32.argtypes = [C.c_float]
        L.orc_bf16_to_f32.restype = C.c_float
        L.orc_bf16_to_f32.argtypes = [C.c_uint16]
        L.orc_bf16_from_f32_n.argtypes = [_f32p, _u16p, _sz]
        for fn in (L.orc_quantize_row_q8_0, L.orc_quantize_row_q4_0):
            fn.argtypes = [_u32p, _u16p, _sz]
        L.orc_quantized_row_words.restype = _sz
        L.orc_quantized_row_words.argtypes = [_sz, C.c_int]
        L.orc_quantize_matrix.argtypes = [_u32p, _u16p, _sz, _sz, C.c_int, C.c_int]
        for fn in (L.orc_gemv_q4, L.orc_gemv_q8):
            fn.argtypes = [_u32p, _f32p, _f32p, _sz, _sz, C.c_int]
        L.orc_gemv_bf16.argtypes = [_u16p, _f32p, _f32p, _sz, _sz]
        L.orc_dot_f32.restype = C.c_float
        L.orc_dot_f32.argtypes = [_f32p, _f32p, _sz]
        L.orc_rmsnorm.argtypes = [_f32p, _f32p, _f32p, _sz, C.c_float]
        L.orc_unit_rmsnorm.argtypes = [_f32p, _f32p, _sz, C.c_float]
        L.orc_gelu_tanh.restype = C.c_float
        L.orc_gelu_tanh.argtypes = [C.c_float]
        L.orc_gate_up_geglu_q4.argtypes = [_f32p, _f32p, _u32p, _u32p, _sz, _sz, C.c_int]
        L.orc_gated_mlp_q4.argtypes = [_f32p, _f32p, _f32p, _u32p, _u32p, _u32p, _sz, _sz, C.c_int]
        L.orc_rope_partial.argtypes = [_f32p, _sz, _sz, _sz, _sz, C.c_float]
        L.orc_softmax.argtypes = [_f32p, _sz]
        L.orc_argmax.restype = C.c_uint32
        L.orc_argmax.argtypes = [_f32p, _sz]
        L.orc_qkv_norm_rope.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz,
                                        _sz, C.c_int, C.c_float, C.c_float, C.c_uint64]
        L.orc_attention.argtypes = [_f32p, _f32p, _f32p, _sz, _u32p, _sz, _sz, _sz, _sz, _f32p]
        L.orc_embed.argtypes = [_u16p, C.c_uint32, _sz, _f32p]
        L.orc_forward_token.restype = C.c_uint32
        L.orc_forward_token.argtypes = [C.c_void_p, _f32p, C.c_uint64, _sz, _u32p, _sz,
                                        C.c_int, _f32p, C.c_int]
        L.orc_forward_layer_batch.restype = C.c_int
        L.orc_forward_layer_batch.argtypes = [C.c_void_p, _sz, _f32p, _sz, C.POINTER(C.c_uint64),
                                              _u32p, _u32p, _sz, _u32p, C.c_int]
        L.orc_gate_mean_sq.restype = C.c_float
        L.orc_gate_mean_sq.argtypes = [_f32p, _f32p, _sz]
        L.orc_forward_token_gated.restype = C.c_uint32
        L.orc_forward_token_gated.argtypes = [C.c_void_p, _f32p, C.c_uint64, _sz, _u32p, _sz,
                                              C.c_int, _f32p, C.c_int, _f32p, C.c_float, _u32p]
        L.orc_qtracker_should_execute.restype = C.c_int
        L.orc_qtracker_should_execute.argtypes = [C.c_void_p, _sz, C.c_uint64, _f32p, _f32p, _sz]
        _lib = L
    return _lib


def _p(a, ct):
    return a.ctypes.data_as(C.POINTER(ct))


def _c(a, dt):
    a = np.ascontiguousarray(a, dtype=dt)
    return a


# ---- bf16 (src/tensor.zig) ----------------------------------------------
def bf16_from_f32(x):
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_bf16_from_f32_n(_p(x, C.c_float), _p(out, C.c_uint16), x.size)
    return out


def bf16_to_f32(b):
    b = _c(b, np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


# ---- quantizers (src/quant.zig) -----------------------------------------
def row_words(cols, mode):
    return lib().orc_quantized_row_words(cols, mode)


def quantize_matrix(w_bf16, mode, nthreads=1):
    w = _c(w_bf16, np.uint16)
    rows, cols = w.shape
    out = np.zeros((rows, row_words(cols, mode)), np.uint32)
    lib().orc_quantize_matrix(_p(out, C.c_uint32), _p(w, C.c_uint16), rows, cols, mode, nthreads)
    return out


def quantize_q4(w_bf16, nthreads=1):
    return quantize_matrix(w_bf16, QUANT_Q4, nthreads)


def quantize_q8(w_bf16, nthreads=1):
    return quantize_matrix(w_bf16, QUANT_Q8, nthreads)


# ---- GEMVs ---------------------------------------------------------------
def gemv_q4(wq, x, cols, nthreads=1):
    wq = _c(wq, np.uint32)
    x = _c(x, np.float32)
    rows = wq.shape[0]
    y = np.empty(rows, np.float32)
    lib().orc_gemv_q4(_p(wq, C.c_uint32), _p(x, C.c_float), _p(y, C.c_float), rows, cols, nthreads)
    return y


def gemv_q8(wq, x, cols, nthreads=1):
    wq = _c(wq, np.uint32)
    x = _c(x, np.float32)
    rows = wq.shape[0]
    y = np.empty(rows, np.float32)
    lib().orc_gemv_q8(_p(wq, C.c_uint32), _p(x, C.c_float), _p(y, C.c_float), rows, cols, nthreads)
    return y


def gemv_bf16(w_bf16, x):
    w = _c(w_bf16, np.uint16)
    x = _c(x, np.float32)
    rows, cols = w.shape
    y = np.empty(rows, np.float32)
    lib().orc_gemv_bf16(_p(w, C.c_uint16), _p(x, C.c_float), _p(y, C.c_float), rows, cols)
    return y


# ---- kernels.zig ---------------------------------------------------------
def dot_f32(a, b):
    a = _c(a, np.float32)
    b = _c(b, np.float32)
    return lib().orc_dot_f32(_p(a, C.c_float), _p(b, C.c_float), min(a.size, b.size))


def rmsnorm(x, w, eps=1e-6):
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    out = np.empty_like(x)
    lib().orc_rmsnorm(_p(out, C.c_float), _p(x, C.c_float), _p(w, C.c_float), x.size, eps)
    return out


def unit_rmsnorm(x, eps=1e-6):
    x = _c(x, np.float32)
    out = np.empty_like(x)
    lib().orc_unit_rmsnorm(_p(out, C.c_float), _p(x, C.c_float), x.size, eps)
    return out


def gelu_tanh(x):
    return lib().orc_gelu_tanh(float(x))


def gate_up_geglu_q4(x, wg, wu, nthreads=1):
    x = _c(x, np.float32)
    wg = _c(wg, np.uint32)
    wu = _c(wu, np.uint32)
    inter = wg.shape[0]
    act = np.empty(inter, np.float32)
    lib().orc_gate_up_geglu_q4(_p(act, C.c_float), _p(x, C.c_float), _p(wg, C.c_uint32),
                               _p(wu, C.c_uint32), inter, x.size, nthreads)
    return act


def gated_mlp_q4(x, wg, wu, wd, nthreads=1):
    x = _c(x, np.float32)
    wg, wu, wd = (_c(a, np.uint32) for a in (wg, wu, wd))
    h, inter = x.size, wg.shape[0]
    act = np.empty(inter, np.float32)
    out = np.empty(h, np.float32)
    lib().orc_gated_mlp_q4(_p(out, C.c_float), _p(act, C.c_float), _p(x, C.c_float),
                           _p(wg, C.c_uint32), _p(wu, C.c_uint32), _p(wd, C.c_uint32),
                           h, inter, nthreads)
    return out, act


def rope_partial(vec, pos, head_dim, rotary_dim, theta):
    v = np.array(vec, dtype=np.float32, copy=True)
    lib().orc_rope_partial(_p(v, C.c_float), v.size, pos, head_dim, rotary_dim, theta)
    return v


def softmax(v):
    v = np.array(v, dtype=np.float32, copy=True)
    lib().orc_softmax(_p(v, C.c_float), v.size)
    return v


def argmax(v):
    v = _c(v, np.float32)
    return int(lib().orc_argmax(_p(v, C.c_float), v.size))


def qkv_norm_rope(q, k, v, q_norm, k_norm, nq, nkv, head_dim, rotary_dim, k_eq_v,
                  theta, eps, clock):
    q = np.array(q, np.float32, copy=True)
    k = np.array(k, np.float32, copy=True)
    v = np.array(v, np.float32, copy=True)
    qn = _c(q_norm, np.float32)
    kn = _c(k_norm, np.float32)
    lib().orc_qkv_norm_rope(_p(q, C.c_float), _p(k, C.c_float), _p(v, C.c_float),
                            _p(qn, C.c_float), _p(kn, C.c_float), nq, nkv, head_dim,
                            rotary_dim, int(k_eq_v), theta, eps, clock)
    return q, k, v


def attention(q, k_cache, v_cache, active, nq, nkv, head_dim):
    """k_cache / v_cache: [slots][nkv*head_dim]."""
    q = _c(q, np.float32)
    kc = _c(k_cache, np.float32)
    vc = _c(v_cache, np.float32)
    act = _c(active, np.uint32)
    out = np.empty(nq * head_dim, np.float32)
    lib().orc_attention(_p(q, C.c_float), _p(kc, C.c_float), _p(vc, C.c_float),
                        nkv * head_dim, _p(act, C.c_uint32), act.size, nq, nkv, head_dim,
                        _p(out, C.c_float))
    return out


def embed(embed_bf16, token, hidden):
    e = _c(embed_bf16, np.uint16)
    x = np.empty(hidden, np.float32)
    lib().orc_embed(_p(e, C.c_uint16), token, hidden, _p(x, C.c_float))
    return x


# ---- layer gating ------------------------------------------------------------
def gate_mean_sq(x, x_prev):
    """quiescence_gate.wgsl's mean (x - x_prev)^2; x_prev (float32) <- x in place."""
    x = _c(x, np.float32)
    assert x_prev.dtype == np.float32 and x_prev.flags.c_contiguous
    return lib().orc_gate_mean_sq(_p(x, C.c_float), _p(x_prev, C.c_float), x.size)


class _QTracker(C.Structure):
    _fields_ = [("enabled", C.c_int), ("split_ratio", C.c_float), ("threshold", C.c_float),
                ("forced_cadence", _sz), ("num_layers", _sz), ("total_evals", C.c_uint64),
                ("skipped_evals", C.c_uint64)]


class QTracker:
    """QuiescenceTracker (src/quiescence.zig:3-61), defaults of QuiescenceConfig."""

    def __init__(self, num_layers, enabled=True, split_ratio=0.5, threshold=0.02,
                 forced_cadence=4):
        self._t = _QTracker(int(enabled), split_ratio, threshold, forced_cadence, num_layers, 0, 0)

    def should_execute(self, layer, clock, x, prev_x):
        x = _c(x, np.float32)
        p = _c(prev_x, np.float32)
        return bool(lib().orc_qtracker_should_execute(C.byref(self._t), layer, clock,
                                                      _p(x, C.c_float), _p(p, C.c_float), x.size))

    @property
    def total_evals(self):
        return self._t.total_evals

    @property
    def skipped_evals(self):
        return self._t.skipped_evals


# ---- ring buffer (src/ring_buffer.zig), a thin Python mirror over C -------
class _Ring(C.Structure):
    _fields_ = [("num_layers", _sz), ("max_kv_dim", _sz), ("num_anchors", _sz),
                ("window_size", _sz), ("num_recall", _sz), ("total_slots", _sz),
                ("k", _f32p), ("v", _f32p), ("clocks", C.POINTER(C.c_uint64)),
                ("active", C.POINTER(C.c_uint8)), ("total_ingested", C.c_uint64)]


class Ring:
    """DynamicRingBuffer (ring_buffer.zig:7-147) backed by the C restatement."""

    def __init__(self, num_layers, max_kv_dim, num_anchors, window_size, num_recall):
        L = lib()
        L.orc_ring_init.restype = C.c_int
        L.orc_ring_init.argtypes = [C.POINTER(_Ring), _sz, _sz, _sz, _sz, _sz]
        L.orc_ring_deinit.argtypes = [C.POINTER(_Ring)]
        L.orc_ring_slot_index.restype = _sz
        L.orc_ring_slot_index.argtypes = [C.POINTER(_Ring), C.c_uint64]
        L.orc_ring_activate_slot.restype = _sz
        L.orc_ring_activate_slot.argtypes = [C.POINTER(_Ring), _sz, C.c_uint64]
        L.orc_ring_write_kv.argtypes = [C.POINTER(_Ring), _sz, C.c_uint64, _f32p, _f32p, _sz]
        L.orc_ring_clear_recall.argtypes = [C.POINTER(_Ring)]
        L.orc_ring_write_recall_kv.argtypes = [C.POINTER(_Ring), _sz, _sz, _f32p, _f32p, _sz,
                                               C.c_uint64]
        L.orc_ring_active_slots.restype = _sz
        L.orc_ring_active_slots.argtypes = [C.POINTER(_Ring), _sz, C.c_uint64, _u32p]
        self._r = _Ring()
        if L.orc_ring_init(C.byref(self._r), num_layers, max_kv_dim, num_anchors,
                           window_size, num_recall) != 0:
            raise MemoryError("ring init failed")

    def __del__(self):
        if getattr(self, "_r", None) is not None and _lib is not None:
            _lib.orc_ring_deinit(C.byref(self._r))
            self._r = None

    @property
    def total_slots(self):
        return self._r.total_slots

    def slot_index(self, clock):
        return lib().orc_ring_slot_index(C.byref(self._r), clock)

    def activate_slot(self, layer, clock):
        return lib().orc_ring_activate_slot(C.byref(self._r), layer, clock)

    def write_kv(self, layer, clock, k, v):
        k = _c(k, np.float32)
        v = _c(v, np.float32)
        lib().orc_ring_write_kv(C.byref(self._r), layer, clock, _p(k, C.c_float),
                                _p(v, C.c_float), k.size)

    def clear_recall(self):
        lib().orc_ring_clear_recall(C.byref(self._r))

    def write_recall_kv(self, layer, rank, k, v, clock):
        k = _c(k, np.float32)
        v = _c(v, np.float32)
        lib().orc_ring_write_recall_kv(C.byref(self._r), layer, rank, _p(k, C.c_float),
                                       _p(v, C.c_float), k.size, clock)

    def active_slots(self, layer, clock):
        out = np.zeros(self.total_slots, np.uint32)
        n = lib().orc_ring_active_slots(C.byref(self._r), layer, clock, _p(out, C.c_uint32))
        return out[:n].copy()


# ---- one decode step -----------------------------------------------------
class _Layer(C.Structure):
    _fields_ = [("full_attention", C.c_int), ("head_dim", _sz), ("rotary_dim", _sz),
                ("num_kv_heads", _sz), ("k_eq_v", C.c_int),
                ("input_norm", _f32p), ("q_norm", _f32p), ("k_norm", _f32p),
                ("post_attn_norm", _f32p), ("pre_ffn_norm", _f32p), ("post_ffn_norm", _f32p),
                ("layer_scalar", C.c_float),
                ("wq", _u32p), ("wk", _u32p), ("wv", _u32p), ("wo", _u32p),
                ("wg", _u32p), ("wu", _u32p), ("wd", _u32p),
                ("k_cache", _f32p), ("v_cache", _f32p)]


class _Model(C.Structure):
    _fields_ = [("hidden", _sz), ("intermediate", _sz), ("vocab", _sz),
                ("num_q_heads", _sz), ("num_layers", _sz), ("layer_mode", C.c_int),
                ("eps", C.c_float), ("rope_theta", C.c_float), ("rope_theta_full", C.c_float),
                ("lm_head", _u32p), ("final_norm", _f32p), ("layers", C.POINTER(_Layer))]


class Model:
    """Quantized weights + per-layer K/V caches for orc_forward_token.

    Matrices and the head are uint32 word arrays: Q4_0 / Q8_0 rows, or in
    layer_mode QUANT_NONE the bf16 rows (two per word) with a bf16 head.

    layers: list of dicts with keys full, head_dim, rotary_dim, num_kv_heads,
    k_eq_v, input_norm, q_norm, k_norm, post_attn_norm, pre_ffn_norm,
    post_ffn_norm, layer_scalar, wq, wk, wv, wo, wg, wu, wd, k_cache, v_cache.
    The numpy arrays are kept alive by this object; k_cache/v_cache are
    updated in place by forward().
    """

    def __init__(self, hidden, intermediate, vocab, num_q_heads, layers, lm_head,
                 final_norm, eps=1e-6, rope_theta=10000.0, rope_theta_full=1e6,
                 layer_mode=QUANT_Q4):
        self._keep = []
        arr = (_Layer * len(layers))()
        for i, d in enumerate(layers):
            L = arr[i]
            L.full_attention = int(d["full"])
            L.head_dim, L.rotary_dim, L.num_kv_heads = d["head_dim"], d["rotary_dim"], d["num_kv_heads"]
            L.k_eq_v = int(d.get("k_eq_v", 0))
            for name in ("input_norm", "q_norm", "k_norm", "post_attn_norm", "pre_ffn_norm",
                         "post_ffn_norm"):
                a = d.get(name)
                if a is None:
                    setattr(L, name, _f32p())
                else:
                    a = _c(a, np.float32)
                    self._keep.append(a)
                    setattr(L, name, _p(a, C.c_float))
            L.layer_scalar = float(d.get("layer_scalar", 1.0))
            for name in ("wq", "wk", "wv", "wo", "wg", "wu", "wd"):
                a = _c(d[name], np.uint32)
                self._keep.append(a)
                setattr(L, name, _p(a, C.c_uint32))
            for name in ("k_cache", "v_cache"):
                a = d[name]
                assert a.dtype == np.float32 and a.flags.c_contiguous
                self._keep.append(a)
                setattr(L, name, _p(a, C.c_float))
        self._layers = arr
        head = _c(lm_head, np.uint32)
        fn = _c(final_norm, np.float32)
        self._keep += [head, fn]
        self._m = _Model(hidden, intermediate, vocab, num_q_heads, len(layers), layer_mode,
                         eps, rope_theta, rope_theta_full, _p(head, C.c_uint32),
                         _p(fn, C.c_float), arr)
        self.vocab = vocab
        self.hidden = hidden

    def forward(self, x, clock, slot_idx, active, want_logits=True, nthreads=1):
        """Returns (token, x_out, logits)."""
        x = np.array(x, np.float32, copy=True)
        act = _c(active, np.uint32)
        logits = np.empty(self.vocab if want_logits else 1, np.float32)
        tok = lib().orc_forward_token(C.byref(self._m), _p(x, C.c_float), clock, slot_idx,
                                      _p(act, C.c_uint32), act.size, int(want_logits),
                                      _p(logits, C.c_float), nthreads)
        return int(tok), x, (logits if want_logits else None)

    def forward_layer_batch(self, layer, X, clocks, slots, actives, nthreads=1):
        """Layer `layer` for T tokens in order (orc_forward_layer_batch): X
        [T][H], token t at clocks[t] in slot slots[t] attending over the
        slot list actives[t].  Returns the layer's outputs [T][H]; the
        layer's caches are updated in place, as T forward() calls on that
        layer alone would leave them (bit for bit)."""
        X = np.array(X, np.float32, copy=True, order="C")
        T = X.shape[0]
        stride = max(1, max(len(a) for a in actives))
        act = np.zeros((T, stride), np.uint32)
        for t, a in enumerate(actives):
            act[t, :len(a)] = a
        n = np.array([len(a) for a in actives], np.uint32)
        ck = np.ascontiguousarray(clocks, np.uint64)
        sl = np.ascontiguousarray(slots, np.uint32)
        rc = lib().orc_forward_layer_batch(C.byref(self._m), layer, _p(X, C.c_float), T,
                                           ck.ctypes.data_as(C.POINTER(C.c_uint64)),
                                           _p(sl, C.c_uint32), _p(act, C.c_uint32), stride,
                                           _p(n, C.c_uint32), nthreads)
        if rc != 0:
            raise MemoryError("orc_forward_layer_batch: out of memory")
        return X

    def forward_gated(self, x, clock, slot_idx, active, x_prev, thresh, want_logits=True,
                      nthreads=1):
        """The gated GPU graph (model_dispatch.zig:45-101); x_prev [L][H]
        float32 is updated in place.  Returns (token, x_out, logits, run)."""
        x = np.array(x, np.float32, copy=True)
        act = _c(active, np.uint32)
        assert x_prev.dtype == np.float32 and x_prev.flags.c_contiguous
        logits = np.empty(self.vocab if want_logits else 1, np.float32)
        run = np.zeros(self._m.num_layers, np.uint32)
        tok = lib().orc_forward_token_gated(C.byref(self._m), _p(x, C.c_float), clock, slot_idx,
                                            _p(act, C.c_uint32), act.size, int(want_logits),
                                            _p(logits, C.c_float), nthreads,
                                            _p(x_prev, C.c_float), thresh,
                                            _p(run, C.c_uint32))
        return int(tok), x, (logits if want_logits else None), run
