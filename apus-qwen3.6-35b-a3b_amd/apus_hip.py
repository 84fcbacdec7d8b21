"""Python binding of libapus_hip.so (the C ABI in include/apus_hip.h).

Tier-1 wrappers take and return numpy arrays (bf16 as uint16 codes, fp32
as float32) and keep the reference's argument meaning (c/gdn.h:107-192,
c/attn.h:87-158). Tier-2 wrappers take torch tensors that live on the GPU
and pass their device pointers; torch is only the allocator here.

Every call raises ApusHipError when the library returns nonzero, so a
missing or failing GPU path is never silently replaced by anything else.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libapus_hip.so")

_u16p = C.POINTER(C.c_uint16)
_f32p = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int32)
_sz = C.c_size_t
_vp = C.c_void_p

# Every symbol include/apus_hip.h declares (checked by the CPU tests).
EXPORTS = [
    "apus_hip_init", "apus_hip_is_enabled", "apus_hip_last_error",
    "apus_hip_set_stream", "apus_hip_synchronize", "apus_hip_malloc",
    "apus_hip_free", "apus_hip_memcpy_h2d", "apus_hip_memcpy_d2h",
    "apus_hip_memset", "apus_hip_timing_enable", "apus_hip_timing_get",
    "apus_hip_gdn_conv1d", "apus_hip_gdn_conv1d_step", "apus_hip_gdn_decay",
    "apus_hip_gdn_beta", "apus_hip_gdn_l2norm", "apus_hip_gdn_step",
    "apus_hip_gdn_step_mt", "apus_hip_gdn_recurrent", "apus_hip_gdn_onorm",
    "apus_hip_attn_rmsnorm", "apus_hip_attn_rope", "apus_hip_attn_gqa",
    "apus_hip_attn_gqa_decode", "apus_hip_attn_gqa_mt",
    "apus_hip_attn_gqa_decode_mt", "apus_hip_attn_outgate",
    "apus_hip_gdn_decode", "apus_hip_gdn_decode_into", "apus_hip_gdn_prefill", "apus_hip_gdn_state_pack", "apus_hip_gdn_state_unpack",
    "apus_hip_attn_cache_pack", "apus_hip_attn_cache_unpack", "apus_hip_attn_decode", "apus_hip_attn_prefill",
    "apus_hip_bf16_gemv", "apus_hip_bf16_gemm", "apus_hip_bf16_weights_release",
    "apus_hip_bf16_gemm_dev", "apus_hip_bf16_gemm_mfma_dev",
    "apus_hip_gdn_decode_slots", "apus_hip_gdn_prefill_slots",
    "apus_hip_attn_cache_pack_paged", "apus_hip_attn_cache_unpack_paged",
    "apus_hip_attn_decode_paged", "apus_hip_attn_prefill_paged",
    "apus_hip_kv_pool_create", "apus_hip_kv_pool_destroy", "apus_hip_kv_pool_cache",
    "apus_hip_kv_seq_open", "apus_hip_kv_seq_reserve", "apus_hip_kv_seq_close",
    "apus_hip_kv_pool_free_blocks",
    "apus_hip_gdn_pool_create", "apus_hip_gdn_pool_destroy", "apus_hip_gdn_pool_state",
    "apus_hip_gdn_slot_open", "apus_hip_gdn_slot_close", "apus_hip_gdn_slot_load",
    "apus_hip_gdn_slot_store",
    "apus_hip_st_open", "apus_hip_st_close", "apus_hip_st_ntensors", "apus_hip_st_find",
    "apus_hip_st_read", "apus_hip_gdn_layer_load", "apus_hip_attn_layer_load",
    "apus_hip_gdn_layer_free", "apus_hip_attn_layer_free", "apus_hip_trace_set",
    "apus_hip_gdn_prefill_noalloc", "apus_hip_set_spin_limit", "apus_hip_attn_split_check",
    "apus_hip_gdn_layer_decode", "apus_hip_gdn_layer_decode_slots",
    "apus_hip_attn_layer_decode", "apus_hip_attn_layer_decode_paged",
]


class ApusHipError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"apus_hip error {code}: {msg}")
        self.code = code


class GdnLayer(C.Structure):
    """ApusHipGdnLayer (include/apus_hip.h)."""
    _fields_ = [("hk", _sz), ("hv", _sz), ("dk", _sz), ("dv", _sz),
                ("conv_w", _vp), ("A_log", _vp), ("dt_bias", _vp),
                ("onorm_w", _vp)]


class KvCache(C.Structure):
    """ApusHipKvCache (include/apus_hip.h): a paged KV cache."""
    _fields_ = [("k", _vp), ("v", _vp), ("block_table", _vp), ("max_blocks", _sz),
                ("max_rows", _sz), ("row_blocks", _vp)]


class AttnLayer(C.Structure):
    """ApusHipAttnLayer (include/apus_hip.h)."""
    _fields_ = [("nh", _sz), ("nkv", _sz), ("d", _sz), ("rot", _sz), ("theta", C.c_double),
                ("qn_w", _vp), ("kn_w", _vp)]


class GdnProj(C.Structure):
    """ApusHipGdnProj (include/apus_hip.h): a GDN layer's projections."""
    _fields_ = [("hidden", _sz), ("w_qkv", _vp), ("w_z", _vp), ("w_b", _vp), ("w_a", _vp),
                ("w_out", _vp)]


class AttnProj(C.Structure):
    """ApusHipAttnProj (include/apus_hip.h): a full-attention layer's
    projections."""
    _fields_ = [("hidden", _sz), ("wq", _vp), ("wk", _vp), ("wv", _vp), ("wo", _vp)]


_lib = None


def load(path=None):
    """Load the library (once). Raises if it was not built. APUS_HIP_LIB
    overrides the path (A/B runs of alternative builds)."""
    global _lib
    path = path or os.environ.get("APUS_HIP_LIB") or LIB_PATH
    if _lib is None:
        # torch ships its own libamdhip64.so.7. Importing it first makes the
        # dynamic loader bind this library to that same HIP runtime (by
        # SONAME), so tensors allocated by torch and our kernels share one
        # runtime; loading ours first would map a second runtime that then
        # hides the GPU from torch.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(path):
            raise FileNotFoundError(
                f"{path} is missing: build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'`")
        _lib = C.CDLL(path)
        for name in EXPORTS:
            getattr(_lib, name).restype = C.c_int
        _lib.apus_hip_last_error.restype = _sz
        _lib.apus_hip_kv_pool_free_blocks.restype = _sz
        _lib.apus_hip_st_ntensors.restype = _sz
    return _lib


def last_error():
    buf = C.create_string_buffer(512)
    load().apus_hip_last_error(buf, 512)
    return buf.value.decode(errors="replace")


def _chk(rc):
    if rc != 0:
        raise ApusHipError(rc, last_error())


def set_spin_limit(polls):
    """Polls a bounded device wait makes before it gives up (0: default)."""
    _chk(load().apus_hip_set_spin_limit(C.c_uint32(int(polls))))


def attn_split_check(cu, pos0, nkv=2, cus=256):
    """Host walk of the decode split plan (apus_hip_attn_split_check):
    returns its 12 counters as a dict."""
    cu = np.ascontiguousarray(cu, np.int32)
    pos0 = np.ascontiguousarray(pos0, np.int32)
    out = np.zeros(12, np.int64)
    _chk(load().apus_hip_attn_split_check(_sz(len(pos0)), cu.ctypes.data_as(_i32p),
                                          pos0.ctypes.data_as(_i32p), _sz(nkv), _sz(cus),
                                          out.ctypes.data_as(C.POINTER(C.c_int64))))
    keys = ("runs", "group_mismatch", "writer_groups", "stream_groups", "bad_keys",
            "bad_slots", "bad_pair_runs", "T1", "pv_runs", "pv_bad_keys", "pv_bad_slots",
            "pv_bad_pair_runs")
    return dict(zip(keys, (int(x) for x in out)))


def _u16(a):
    assert a.dtype == np.uint16 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_u16p)


def _f32(a):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_f32p)


def _dp(t):
    """Device pointer of a torch tensor (or None)."""
    if t is None:
        return None
    assert t.is_cuda and t.is_contiguous(), "tier-2 tensors must be contiguous GPU tensors"
    return _vp(t.data_ptr())


def init(device=0):
    err = C.create_string_buffer(512)
    rc = load().apus_hip_init(C.c_int(device), err, 512)
    if rc != 0:
        raise ApusHipError(rc, err.value.decode(errors="replace"))


def set_stream(stream_handle):
    _chk(load().apus_hip_set_stream(_vp(stream_handle)))


def synchronize():
    _chk(load().apus_hip_synchronize())


def timing_enable(on=True):
    _chk(load().apus_hip_timing_enable(C.c_int(1 if on else 0)))


def timing_get(kernel):
    """(total milliseconds, launches) recorded for one kernel name."""
    ms = C.c_double(0.0)
    n = _sz(0)
    _chk(load().apus_hip_timing_get(kernel.encode(), C.byref(ms), C.byref(n)))
    return ms.value, n.value


# ---------------------------------------------------------------- tier 1
def gdn_conv1d(x, w, state):
    T, Cc = x.shape
    out = np.empty_like(x)
    _chk(load().apus_hip_gdn_conv1d(_u16(x), _u16(w), _u16(out), _sz(Cc),
                                    _sz(T), _u16(state)))
    return out


def gdn_conv1d_step(x, w, state):
    out = np.empty_like(x)
    _chk(load().apus_hip_gdn_conv1d_step(_u16(x), _u16(w), _u16(out),
                                         _sz(x.size), _u16(state)))
    return out


def gdn_decay(a, A_log, dt_bias):
    g = np.empty(a.size, np.float32)
    _chk(load().apus_hip_gdn_decay(_u16(a), _f32(A_log), _f32(dt_bias),
                                   _f32(g), _sz(a.size)))
    return g


def gdn_beta(b):
    beta = np.empty_like(b)
    _chk(load().apus_hip_gdn_beta(_u16(b), _u16(beta), _sz(b.size)))
    return beta


def gdn_l2norm(x, H, D, scale):
    y = np.empty(H * D, np.float32)
    _chk(load().apus_hip_gdn_l2norm(_u16(x), _f32(y), _sz(H), _sz(D),
                                    C.c_float(scale)))
    return y


def gdn_step(S, q, k, v, g, beta, H, Dk, Dv):
    o = np.empty(H * Dv, np.float32)
    _chk(load().apus_hip_gdn_step(_f32(S), _f32(q), _f32(k), _u16(v), _f32(g),
                                  _u16(beta), _f32(o), _sz(H), _sz(Dk),
                                  _sz(Dv)))
    return o


def gdn_step_mt(S, q, k, v, g, beta, H, Dk, Dv):
    o = np.empty(H * Dv, np.float32)
    _chk(load().apus_hip_gdn_step_mt(_f32(S), _f32(q), _f32(k), _u16(v),
                                     _f32(g), _u16(beta), _f32(o), _sz(H),
                                     _sz(Dk), _sz(Dv)))
    return o


def gdn_recurrent(S, q, k, v, g, beta, T, H, Dk, Dv):
    o = np.empty(T * H * Dv, np.float32)
    _chk(load().apus_hip_gdn_recurrent(_f32(S), _f32(q), _f32(k), _u16(v),
                                       _f32(g), _u16(beta), _f32(o), _sz(T),
                                       _sz(H), _sz(Dk), _sz(Dv)))
    return o


def gdn_onorm(o, z, w, H, D):
    y = np.empty(H * D, np.uint16)
    _chk(load().apus_hip_gdn_onorm(_u16(o), _u16(z), _u16(w), _u16(y),
                                   _sz(H), _sz(D)))
    return y


def attn_rmsnorm(x, w):
    y = np.empty_like(x)
    _chk(load().apus_hip_attn_rmsnorm(_u16(x), _u16(w), _u16(y), _sz(x.size)))
    return y


def attn_rope(x, rot, pos, theta=1e7):
    y = np.empty_like(x)
    _chk(load().apus_hip_attn_rope(_u16(x), _u16(y), _sz(x.size), _sz(rot),
                                   C.c_float(pos), C.c_double(theta)))
    return y


def attn_gqa(q, kc, vc, Tq, Tk, H, Hkv, D, scale):
    o = np.empty(Tq * H * D, np.uint16)
    _chk(load().apus_hip_attn_gqa(_u16(q), _u16(kc), _u16(vc), _u16(o),
                                  _sz(Tq), _sz(Tk), _sz(H), _sz(Hkv), _sz(D),
                                  C.c_float(scale), None, None))
    return o


def attn_gqa_decode(q, kc, vc, Tk, H, Hkv, D, scale):
    o = np.empty(H * D, np.uint16)
    _chk(load().apus_hip_attn_gqa_decode(_u16(q), _u16(kc), _u16(vc), _u16(o),
                                         _sz(Tk), _sz(H), _sz(Hkv), _sz(D),
                                         C.c_float(scale), None, None))
    return o


def attn_gqa_mt(q, kc, vc, Tq, Tk, H, Hkv, D, scale):
    o = np.empty(Tq * H * D, np.uint16)
    _chk(load().apus_hip_attn_gqa_mt(_u16(q), _u16(kc), _u16(vc), _u16(o),
                                     _sz(Tq), _sz(Tk), _sz(H), _sz(Hkv),
                                     _sz(D), C.c_float(scale)))
    return o


def attn_outgate(o, gate):
    y = np.empty_like(o)
    _chk(load().apus_hip_attn_outgate(_u16(o), _u16(gate), _u16(y),
                                      _sz(o.size)))
    return y


# ---------------------------------------------------------------- tier 2
def _cu_arr(cu):
    cu = np.ascontiguousarray(np.asarray(cu, dtype=np.int32))
    return cu, cu.ctypes.data_as(_i32p), len(cu) - 1


def gdn_layer(dims, w):
    """Build an ApusHipGdnLayer from dims (hk, hv, dk, dv) and a dict of
    device tensors conv_w, A_log, dt_bias, onorm_w. The struct carries raw
    device pointers, so it keeps a reference to the tensors: they stay
    allocated as long as the layer object lives."""
    hk, hv, dk, dv = dims
    for k in ("conv_w", "A_log", "dt_bias", "onorm_w"):
        assert w[k].is_cuda and w[k].is_contiguous(), k
    layer = GdnLayer(hk, hv, dk, dv, w["conv_w"].data_ptr(),
                     w["A_log"].data_ptr(), w["dt_bias"].data_ptr(),
                     w["onorm_w"].data_ptr())
    layer._tensors = dict(w)
    return layer


def gdn_decode(layer, cu, qkv, z, a, b, conv_state, S, y):
    cu, cup, B = _cu_arr(cu)
    _chk(load().apus_hip_gdn_decode(C.byref(layer), _sz(B), cup, _dp(qkv),
                                    _dp(z), _dp(a), _dp(b), _dp(conv_state),
                                    _dp(S), _dp(y)))


class BoundCall:
    """One library call with its arguments converted once. Calling it
    repeats the call on the same buffers and host arrays (kept alive here):
    for a loop that re-runs one step, it leaves only the foreign-function
    call itself on the host path."""
    __slots__ = ("_f", "_args", "_keep")

    def __init__(self, f, args, keep):
        self._f, self._args, self._keep = f, args, keep

    def __call__(self):
        rc = self._f(*self._args)
        if rc != 0:
            raise ApusHipError(rc, last_error())


def gdn_decode_bound(layer, cu, qkv, z, a, b, conv_state, S, y):
    """gdn_decode as a BoundCall."""
    cu, cup, B = _cu_arr(cu)
    args = (C.byref(layer), _sz(B), cup, _dp(qkv), _dp(z), _dp(a), _dp(b), _dp(conv_state),
            _dp(S), _dp(y))
    return BoundCall(load().apus_hip_gdn_decode, args, (layer, cu, qkv, z, a, b, conv_state, S, y))


def gdn_decode_into(layer, cu, qkv, z, a, b, conv_in, S_in, conv_out, S_out, y):
    """Out-of-place decode/verify: states read from (conv_in, S_in), written
    to (conv_out, S_out); sequences with no tokens are left untouched."""
    cu, cup, B = _cu_arr(cu)
    _chk(load().apus_hip_gdn_decode_into(C.byref(layer), _sz(B), cup, _dp(qkv),
                                         _dp(z), _dp(a), _dp(b), _dp(conv_in),
                                         _dp(S_in), _dp(conv_out), _dp(S_out),
                                         _dp(y)))


def gdn_prefill(layer, cu, qkv, z, a, b, conv_state, S, y):
    """Chunked prefill; arguments as gdn_decode (device tensors)."""
    cu, cup, B = _cu_arr(cu)
    _chk(load().apus_hip_gdn_prefill(C.byref(layer), _sz(B), cup, _dp(qkv),
                                     _dp(z), _dp(a), _dp(b), _dp(conv_state),
                                     _dp(S), _dp(y)))


def gdn_prefill_noalloc(layer, cu, qkv, z, a, b, conv_state, S, y):
    """apus_hip_gdn_prefill_noalloc: the chunked prefill in the library's
    fixed per-device scratch (allocates nothing)."""
    cu, cup, B = _cu_arr(cu)
    _chk(load().apus_hip_gdn_prefill_noalloc(C.byref(layer), _sz(B), cup, _dp(qkv), _dp(z),
                                             _dp(a), _dp(b), _dp(conv_state), _dp(S), _dp(y)))


def gdn_state_pack(S_ref, S_dev):
    """Reference-layout states [n, 128, 128] -> device layout (GPU tensors)."""
    _chk(load().apus_hip_gdn_state_pack(_dp(S_ref), _dp(S_dev), _sz(S_ref.numel() // (128 * 128))))


def gdn_state_unpack(S_dev, S_ref):
    _chk(load().apus_hip_gdn_state_unpack(_dp(S_dev), _dp(S_ref), _sz(S_dev.numel() // (128 * 128))))


def attn_layer(dims, w):
    """ApusHipAttnLayer from dims (nh, nkv, d, rot, theta) and device tensors
    qn_w, kn_w; the layer keeps a reference to them (raw device pointers)."""
    nh, nkv, d, rot, theta = dims
    for k in ("qn_w", "kn_w"):
        assert w[k].is_cuda and w[k].is_contiguous(), k
    layer = AttnLayer(nh, nkv, d, rot, theta, w["qn_w"].data_ptr(), w["kn_w"].data_ptr())
    layer._tensors = dict(w)
    return layer


def attn_cache_pack(kc_ref, vc_ref, ntok, nkv, d, kcache, vcache, max_seq):
    """One sequence: reference-layout caches [ntok, nkv, d] -> device layout."""
    _chk(load().apus_hip_attn_cache_pack(_dp(kc_ref), _dp(vc_ref), _sz(ntok), _sz(nkv), _sz(d),
                                         _dp(kcache), _dp(vcache), _sz(max_seq)))


def attn_cache_unpack(kcache, vcache, ntok, nkv, d, max_seq, kc_ref, vc_ref):
    _chk(load().apus_hip_attn_cache_unpack(_dp(kcache), _dp(vcache), _sz(ntok), _sz(nkv), _sz(d),
                                           _sz(max_seq), _dp(kc_ref), _dp(vc_ref)))


def attn_decode(layer, cu, pos0, qg, k, v, kcache, vcache, max_seq, y):
    cu, cup, B = _cu_arr(cu)
    pos0 = np.ascontiguousarray(np.asarray(pos0, dtype=np.int32))
    _chk(load().apus_hip_attn_decode(C.byref(layer), _sz(B), cup, pos0.ctypes.data_as(_i32p),
                                     _dp(qg), _dp(k), _dp(v), _dp(kcache), _dp(vcache),
                                     _sz(max_seq), _dp(y)))


def attn_prefill(layer, cu, pos0, qg, k, v, kcache, vcache, max_seq, y):
    """Causal prefill of any number of new tokens per sequence; arguments
    as attn_decode."""
    cu, cup, B = _cu_arr(cu)
    pos0 = np.ascontiguousarray(np.asarray(pos0, dtype=np.int32))
    _chk(load().apus_hip_attn_prefill(C.byref(layer), _sz(B), cup, pos0.ctypes.data_as(_i32p),
                                      _dp(qg), _dp(k), _dp(v), _dp(kcache), _dp(vcache),
                                      _sz(max_seq), _dp(y)))


# ---- projections (c/bf16.h:178-231)
def bf16_gemv(w, x):
    """Drop-in of the reference's bf16_gemv hook: numpy w [O,K], x [K]
    (uint16 codes) -> y [O]. Bitwise the reference's order."""
    O, K = w.shape
    y = np.empty(O, np.uint16)
    _chk(load().apus_hip_bf16_gemv(_u16(w), _u16(x), _u16(y), _sz(O), _sz(K)))
    return y


def bf16_gemm(w, x):
    """Drop-in of the bf16_gemm hook: w [O,K], x [M,K] -> y [M,O]."""
    O, K = w.shape
    M = x.shape[0]
    y = np.empty((M, O), np.uint16)
    _chk(load().apus_hip_bf16_gemm(_u16(w), _u16(x), _u16(y), _sz(M), _sz(O), _sz(K)))
    return y


def bf16_weights_release():
    _chk(load().apus_hip_bf16_weights_release())


def bf16_gemm_dev(w, x, y, exact=True):
    """Device tensors (int16 views of bf16 codes): w [O,K], x [M,K],
    y [M,O]. exact: the reference's order (bitwise); else the MFMA GEMM."""
    O, K = w.shape
    M = x.shape[0]
    f = load().apus_hip_bf16_gemm_dev if exact else load().apus_hip_bf16_gemm_mfma_dev
    _chk(f(_dp(w), _dp(x), _dp(y), _sz(M), _sz(O), _sz(K)))


# ---- paged KV cache and state pools
def _i32arr(x):
    x = np.ascontiguousarray(np.asarray(x, dtype=np.int32))
    return x, x.ctypes.data_as(_i32p)


def attn_decode_paged(layer, rows, cu, pos0, qg, k, v, kv, y):
    """Decode on a paged cache: kv is a KvCache, rows the block-table row of
    each sequence (host)."""
    cu, cup, B = _cu_arr(cu)
    rows, rp = _i32arr(rows)
    pos0, pp = _i32arr(pos0)
    _chk(load().apus_hip_attn_decode_paged(C.byref(layer), _sz(B), rp, cup, pp, _dp(qg), _dp(k),
                                           _dp(v), C.byref(kv), _dp(y)))


def attn_prefill_paged(layer, rows, cu, pos0, qg, k, v, kv, y):
    cu, cup, B = _cu_arr(cu)
    rows, rp = _i32arr(rows)
    pos0, pp = _i32arr(pos0)
    _chk(load().apus_hip_attn_prefill_paged(C.byref(layer), _sz(B), rp, cup, pp, _dp(qg), _dp(k),
                                            _dp(v), C.byref(kv), _dp(y)))


def attn_cache_pack_paged(kc_ref, vc_ref, ntok, nkv, d, kv, row):
    _chk(load().apus_hip_attn_cache_pack_paged(_dp(kc_ref), _dp(vc_ref), _sz(ntok), _sz(nkv),
                                               _sz(d), C.byref(kv), C.c_int32(row)))


def attn_cache_unpack_paged(kv, row, ntok, nkv, d, kc_ref, vc_ref):
    _chk(load().apus_hip_attn_cache_unpack_paged(C.byref(kv), C.c_int32(row), _sz(ntok), _sz(nkv),
                                                 _sz(d), _dp(kc_ref), _dp(vc_ref)))


def gdn_decode_slots(layer, slot_in, slot_out, cu, qkv, z, a, b, conv, S, y):
    cu, cup, B = _cu_arr(cu)
    si, sip = _i32arr(slot_in)
    so, sop = _i32arr(slot_out)
    _chk(load().apus_hip_gdn_decode_slots(C.byref(layer), _sz(B), sip, sop, cup, _dp(qkv), _dp(z),
                                          _dp(a), _dp(b), C.c_void_p(conv), C.c_void_p(S),
                                          _dp(y)))


def gdn_proj(hidden, w):
    """ApusHipGdnProj from a dict of device tensors w_qkv, w_z, w_b, w_a,
    w_out (int16 views of bf16, reference layouts); keeps them alive."""
    for k in ("w_qkv", "w_z", "w_b", "w_a", "w_out"):
        assert w[k].is_cuda and w[k].is_contiguous(), k
    p = GdnProj(hidden, w["w_qkv"].data_ptr(), w["w_z"].data_ptr(), w["w_b"].data_ptr(),
                w["w_a"].data_ptr(), w["w_out"].data_ptr())
    p._tensors = dict(w)
    return p


def attn_proj(hidden, w):
    """ApusHipAttnProj from device tensors wq, wk, wv, wo."""
    for k in ("wq", "wk", "wv", "wo"):
        assert w[k].is_cuda and w[k].is_contiguous(), k
    p = AttnProj(hidden, w["wq"].data_ptr(), w["wk"].data_ptr(), w["wv"].data_ptr(),
                 w["wo"].data_ptr())
    p._tensors = dict(w)
    return p


def gdn_layer_decode(layer, proj, cu, ln1, conv, S, ao):
    """GDN layer with projections: ln1 [T, H] -> ao [T, H] (flat states)."""
    cu, cup, B = _cu_arr(cu)
    _chk(load().apus_hip_gdn_layer_decode(C.byref(layer), C.byref(proj), _sz(B), cup, _dp(ln1),
                                          _dp(conv), _dp(S), _dp(ao)))


def gdn_layer_decode_slots(layer, proj, slot_in, slot_out, cu, ln1, conv, S, ao):
    """As gdn_layer_decode on a state pool (conv, S: the slot arrays' base
    addresses as ints)."""
    cu, cup, B = _cu_arr(cu)
    si, sip = _i32arr(slot_in)
    so, sop = _i32arr(slot_out)
    _chk(load().apus_hip_gdn_layer_decode_slots(C.byref(layer), C.byref(proj), _sz(B), sip, sop,
                                                cup, _dp(ln1), C.c_void_p(conv), C.c_void_p(S),
                                                _dp(ao)))


def attn_layer_decode(layer, proj, cu, pos0, ln1, kcache, vcache, max_seq, ao):
    """Full-attention layer with projections on a flat cache."""
    cu, cup, B = _cu_arr(cu)
    pos0, pp = _i32arr(pos0)
    _chk(load().apus_hip_attn_layer_decode(C.byref(layer), C.byref(proj), _sz(B), cup, pp,
                                           _dp(ln1), _dp(kcache), _dp(vcache), _sz(max_seq),
                                           _dp(ao)))


def attn_layer_decode_paged(layer, proj, rows, cu, pos0, ln1, kv, ao):
    """Full-attention layer with projections on a paged cache."""
    cu, cup, B = _cu_arr(cu)
    rows, rp = _i32arr(rows)
    pos0, pp = _i32arr(pos0)
    _chk(load().apus_hip_attn_layer_decode_paged(C.byref(layer), C.byref(proj), _sz(B), rp, cup,
                                                 pp, _dp(ln1), C.byref(kv), _dp(ao)))


def gdn_prefill_slots(layer, slots, cu, qkv, z, a, b, conv, S, y):
    cu, cup, B = _cu_arr(cu)
    sl, slp = _i32arr(slots)
    _chk(load().apus_hip_gdn_prefill_slots(C.byref(layer), _sz(B), slp, cup, _dp(qkv), _dp(z),
                                           _dp(a), _dp(b), C.c_void_p(conv), C.c_void_p(S),
                                           _dp(y)))


class KvPool:
    """apus_hip_kv_pool_*: a paged KV cache shared by nlayers layers."""

    def __init__(self, nlayers, nkv, d, nblocks, max_rows, max_blocks):
        self.h = C.c_void_p()
        _chk(load().apus_hip_kv_pool_create(_sz(nlayers), _sz(nkv), _sz(d), _sz(nblocks),
                                            _sz(max_rows), _sz(max_blocks), C.byref(self.h)))

    def cache(self, layer):
        kv = KvCache()
        _chk(load().apus_hip_kv_pool_cache(self.h, _sz(layer), C.byref(kv)))
        return kv

    def open(self):
        r = C.c_int32()
        _chk(load().apus_hip_kv_seq_open(self.h, C.byref(r)))
        return r.value

    def reserve(self, row, ntok):
        _chk(load().apus_hip_kv_seq_reserve(self.h, C.c_int32(row), _sz(ntok)))

    def close(self, row):
        _chk(load().apus_hip_kv_seq_close(self.h, C.c_int32(row)))

    def free_blocks(self):
        return load().apus_hip_kv_pool_free_blocks(self.h)

    def destroy(self):
        if self.h:
            _chk(load().apus_hip_kv_pool_destroy(self.h))
            self.h = C.c_void_p()


class GdnPool:
    """apus_hip_gdn_pool_*: per-sequence GDN states for nlayers layers."""

    def __init__(self, nlayers, dims, nslots):
        hk, hv, dk, dv = dims
        self.h = C.c_void_p()
        _chk(load().apus_hip_gdn_pool_create(_sz(nlayers), _sz(hk), _sz(hv), _sz(dk), _sz(dv),
                                             _sz(nslots), C.byref(self.h)))

    def state(self, layer):
        """(conv, S) device base addresses of the layer's slot arrays."""
        conv, S = C.c_void_p(), C.c_void_p()
        _chk(load().apus_hip_gdn_pool_state(self.h, _sz(layer), C.byref(conv), C.byref(S)))
        return conv.value, S.value

    def open(self):
        r = C.c_int32()
        _chk(load().apus_hip_gdn_slot_open(self.h, C.byref(r)))
        return r.value

    def close(self, slot):
        _chk(load().apus_hip_gdn_slot_close(self.h, C.c_int32(slot)))

    def load_state(self, layer, slot, conv, S):
        """Import one sequence's state (device tensors, reference layout:
        conv [conv_dim*3] codes, S [hv, dk, dv] f32) into a slot."""
        _chk(load().apus_hip_gdn_slot_load(self.h, _sz(layer), C.c_int32(slot), _dp(conv), _dp(S)))

    def store_state(self, layer, slot, conv, S):
        _chk(load().apus_hip_gdn_slot_store(self.h, _sz(layer), C.c_int32(slot), _dp(conv), _dp(S)))

    def destroy(self):
        if self.h:
            _chk(load().apus_hip_gdn_pool_destroy(self.h))
            self.h = C.c_void_p()


# ---- weight container reader
ST_DTYPES = {0: "I8", 1: "U8", 2: "F8_E8M0", 3: "F8_E4M3", 4: "BF16", 5: "F16", 6: "F32",
             7: "I32", 8: "I64", 9: "OTHER"}


class StTensor(C.Structure):
    """ApusHipStTensor (include/apus_hip.h)."""
    _fields_ = [("name", C.c_char * 160), ("dtype", C.c_int), ("ndim", C.c_int),
                ("shape", C.c_int64 * 8), ("nbytes", _sz)]


class Container:
    """apus_hip_st_*: a safetensors shard or a directory with
    model.safetensors.index.json (host-side; no device needed)."""

    def __init__(self, path):
        self.h = C.c_void_p()
        _chk(load().apus_hip_st_open(os.fsencode(path), C.byref(self.h)))

    def __len__(self):
        return load().apus_hip_st_ntensors(self.h)

    def find(self, name):
        t = StTensor()
        _chk(load().apus_hip_st_find(self.h, name.encode(), C.byref(t)))
        return dict(name=t.name.decode(), dtype=ST_DTYPES[t.dtype],
                    shape=tuple(t.shape[i] for i in range(t.ndim)), nbytes=t.nbytes)

    def read(self, name):
        """The payload as raw bytes (numpy uint8)."""
        info = self.find(name)
        buf = np.empty(info["nbytes"], np.uint8)
        _chk(load().apus_hip_st_read(self.h, name.encode(), buf.ctypes.data_as(_vp),
                                     _sz(buf.size)))
        return buf

    def gdn_layer(self, layer, dims):
        """GdnLayer with device copies of layer `layer`'s weights (free with
        free_gdn_layer)."""
        hk, hv, dk, dv = dims
        L = GdnLayer()
        _chk(load().apus_hip_gdn_layer_load(self.h, C.c_int(layer), _sz(hk), _sz(hv), _sz(dk),
                                            _sz(dv), C.byref(L)))
        return L

    def attn_layer(self, layer, dims):
        nh, nkv, d, rot, theta = dims
        L = AttnLayer()
        _chk(load().apus_hip_attn_layer_load(self.h, C.c_int(layer), _sz(nh), _sz(nkv), _sz(d),
                                             _sz(rot), C.c_double(theta), C.byref(L)))
        return L

    def close(self):
        if self.h:
            _chk(load().apus_hip_st_close(self.h))
            self.h = C.c_void_p()


def free_gdn_layer(L):
    _chk(load().apus_hip_gdn_layer_free(C.byref(L)))


def free_attn_layer(L):
    _chk(load().apus_hip_attn_layer_free(C.byref(L)))


# ---- named-intermediate capture
class GdnTrace(C.Structure):
    """ApusHipGdnTrace (include/apus_hip.h)."""
    _fields_ = [("qkv_conv", _vp), ("beta", _vp), ("gdecay", _vp), ("rec_o", _vp),
                ("onorm", _vp)]


class AttnTrace(C.Structure):
    """ApusHipAttnTrace (include/apus_hip.h)."""
    _fields_ = [("qf", _vp), ("kf", _vp), ("attno", _vp), ("mgate", _vp)]


def trace_set(gdn=None, attn=None):
    """gdn / attn: dicts of device tensors by field name (missing fields are
    not captured), or None to stop tracing that mixer."""
    def mk(cls, d):
        if d is None:
            return None
        return cls(*[_dp(d.get(f)) for f, _ in cls._fields_])
    g, a = mk(GdnTrace, gdn), mk(AttnTrace, attn)
    trace_set._keep = (gdn, attn)      # the tensors must outlive the trace
    _chk(load().apus_hip_trace_set(C.byref(g) if g is not None else None,
                                   C.byref(a) if a is not None else None))
