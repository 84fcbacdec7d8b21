"""ctypes front-end for the CPU oracle (oracle/liboracle.so) and, when it
was built, the reference anchors (oracle/_ref/libapus_ref.so).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg. Arrays are numpy: bf16 travels as uint16
codes, fp32 as float32, exactly like the reference's C signatures
(c/gdn.h:107-192, c/attn.h:87-158).
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libapus_ref.so")

_u16p = C.POINTER(C.c_uint16)
_f32p = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int32)
_sz = C.c_size_t


def _p(a, typ):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "arrays must be C-contiguous"
    return a.ctypes.data_as(typ)


def u16(a):
    return _p(a, _u16p)


def f32(a):
    return _p(a, _f32p)


def i32(a):
    return _p(a, _i32p)


class _GdnDims(C.Structure):
    _fields_ = [("hk", _sz), ("hv", _sz), ("dk", _sz), ("dv", _sz)]


class _AttnDims(C.Structure):
    _fields_ = [("nh", _sz), ("nkv", _sz), ("d", _sz), ("rot", _sz),
                ("theta", C.c_double)]


class _GdnTrace(C.Structure):
    _fields_ = [("qkv_conv", _u16p), ("beta", _u16p), ("gdecay", _f32p),
                ("rec_o", _u16p)]


def _load(path):
    if not os.path.exists(path):
        raise FileNotFoundError(
            f"{path} is not built; run `make -C oracle` (and `make -C oracle ref`)")
    return C.CDLL(path)


class _Ops:
    """Per-op wrappers shared by the oracle and the reference library.

    `pre` is the C symbol prefix: "orc_" for the oracle, "apus_" for the
    reference anchors (same argument lists, c/gdn.h and c/attn.h)."""

    def __init__(self, lib, pre):
        self.lib, self.pre = lib, pre

    def _f(self, name):
        return getattr(self.lib, self.pre + name)

    # --- GDN -----------------------------------------------------------
    def gdn_conv1d(self, x, w, state):
        T, Cc = x.shape
        out = np.empty_like(x)
        self._f("gdn_conv1d")(u16(x), u16(w), u16(out), _sz(Cc), _sz(T),
                              u16(state))
        return out

    def gdn_conv1d_step(self, x, w, state):
        out = np.empty_like(x)
        self._f("gdn_conv1d_step")(u16(x), u16(w), u16(out), _sz(x.size),
                                   u16(state))
        return out

    def gdn_decay(self, a, A_log, dt_bias):
        g = np.empty(a.size, np.float32)
        self._f("gdn_decay")(u16(a), f32(A_log), f32(dt_bias), f32(g),
                             _sz(a.size))
        return g

    def gdn_beta(self, b):
        beta = np.empty_like(b)
        self._f("gdn_beta")(u16(b), u16(beta), _sz(b.size))
        return beta

    def gdn_l2norm(self, x, H, D, scale):
        y = np.empty(H * D, np.float32)
        self._f("gdn_l2norm")(u16(x), f32(y), _sz(H), _sz(D),
                              C.c_float(scale))
        return y

    def gdn_step(self, S, q, k, v, g, beta, H, Dk, Dv):
        o = np.empty(H * Dv, np.float32)
        self._f("gdn_step")(f32(S), f32(q), f32(k), u16(v), f32(g), u16(beta),
                            f32(o), _sz(H), _sz(Dk), _sz(Dv))
        return o

    def gdn_recurrent(self, S, q, k, v, g, beta, T, H, Dk, Dv):
        o = np.empty(T * H * Dv, np.float32)
        self._f("gdn_recurrent")(f32(S), f32(q), f32(k), u16(v), f32(g),
                                 u16(beta), f32(o), _sz(T), _sz(H), _sz(Dk),
                                 _sz(Dv))
        return o

    def gdn_onorm(self, o, z, w, H, D):
        y = np.empty(H * D, np.uint16)
        self._f("gdn_onorm")(u16(o), u16(z), u16(w), u16(y), _sz(H), _sz(D))
        return y

    # --- attention -----------------------------------------------------
    def attn_rmsnorm(self, x, w):
        y = np.empty_like(x)
        self._f("attn_rmsnorm")(u16(x), u16(w), u16(y), _sz(x.size))
        return y

    def attn_rope(self, x, rot, pos, theta=1e7):
        y = np.empty_like(x)
        self._f("attn_rope")(u16(x), u16(y), _sz(x.size), _sz(rot),
                             C.c_float(pos), C.c_double(theta))
        return y

    def attn_gqa(self, q, kc, vc, Tq, Tk, H, Hkv, D, scale):
        o = np.empty(Tq * H * D, np.uint16)
        ab = np.empty(Tk, np.uint16)
        eb = np.empty(Tk, np.float32)
        self._f("attn_gqa")(u16(q), u16(kc), u16(vc), u16(o), _sz(Tq),
                            _sz(Tk), _sz(H), _sz(Hkv), _sz(D),
                            C.c_float(scale), u16(ab), f32(eb))
        return o

    def attn_outgate(self, o, gate):
        y = np.empty_like(o)
        self._f("attn_outgate")(u16(o), u16(gate), u16(y), _sz(o.size))
        return y


class Oracle(_Ops):
    """The repo's own C restatement (oracle/apus_oracle.c)."""

    def __init__(self):
        super().__init__(_load(ORACLE_SO), "orc_")
        L = self.lib
        L.orc_bf16_bits.restype = C.c_uint16
        L.orc_bf16_bits.argtypes = [C.c_float]
        L.orc_bf16_f32.restype = C.c_float
        L.orc_bf16_f32.argtypes = [C.c_uint16]
        L.orc_max_threads.restype = C.c_int

    def bf16_narrow(self, x):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(x.shape, np.uint16)
        self.lib.orc_bf16_narrow(f32(x), u16(y), _sz(x.size))
        return y

    def max_threads(self):
        return self.lib.orc_max_threads()

    def gdn_step_mt(self, S, q, k, v, g, beta, H, Dk, Dv, nthreads=0):
        o = np.empty(H * Dv, np.float32)
        self.lib.orc_gdn_step_mt(f32(S), f32(q), f32(k), u16(v), f32(g),
                                 u16(beta), f32(o), _sz(H), _sz(Dk), _sz(Dv),
                                 C.c_int(nthreads))
        return o

    def attn_gqa_mt(self, q, kc, vc, Tq, Tk, H, Hkv, D, scale, nthreads=0):
        o = np.empty(Tq * H * D, np.uint16)
        self.lib.orc_attn_gqa_mt(u16(q), u16(kc), u16(vc), u16(o), _sz(Tq),
                                 _sz(Tk), _sz(H), _sz(Hkv), _sz(D),
                                 C.c_float(scale), C.c_int(nthreads))
        return o

    def rope_table(self, pos, rot, theta=1e7):
        cs = np.empty(rot, np.uint16)
        self.lib.orc_attn_rope_table(C.c_float(pos), _sz(rot),
                                     C.c_double(theta), u16(cs))
        return cs

    def gdn_mixer(self, dims, w, cu, qkv, z, a, b, conv_state, S,
                  nthreads=0, trace=False):
        """dims = (hk, hv, dk, dv); w = dict(conv_w, A_log, dt_bias, onorm_w).
        conv_state and S are updated in place. Returns y (and the trace)."""
        hk, hv, dk, dv = dims
        B = len(cu) - 1
        Ttot = int(cu[-1])
        y = np.empty((Ttot, hv * dv), np.uint16)
        tr = None
        trd = None
        if trace:
            cd = 2 * hk * dk + hv * dv
            trd = dict(qkv_conv=np.empty((Ttot, cd), np.uint16),
                       beta=np.empty((Ttot, hv), np.uint16),
                       gdecay=np.empty((Ttot, hv), np.float32),
                       rec_o=np.empty((Ttot, hv * dv), np.uint16))
            tr = C.byref(_GdnTrace(u16(trd["qkv_conv"]), u16(trd["beta"]),
                                   f32(trd["gdecay"]), u16(trd["rec_o"])))
        self.lib.orc_gdn_mixer(C.byref(_GdnDims(hk, hv, dk, dv)),
                               u16(w["conv_w"]), f32(w["A_log"]),
                               f32(w["dt_bias"]), u16(w["onorm_w"]), _sz(B),
                               i32(cu), u16(qkv), u16(z), u16(a), u16(b),
                               u16(conv_state), f32(S), u16(y), tr,
                               C.c_int(nthreads))
        return (y, trd) if trace else y

    def bf16_gemm(self, w, x):
        """w [O,K], x [M,K] (uint16 codes) -> y [M,O] (c/bf16.h:285-300)."""
        O, K = w.shape
        M = x.shape[0]
        y = np.empty((M, O), np.uint16)
        self.lib.orc_bf16_gemm(u16(w), u16(x), u16(y), _sz(M), _sz(O), _sz(K))
        return y

    def attn_mixer(self, dims, w, cu, pos0, qg, k, v, kcache, vcache,
                   cache_stride, nthreads=0, capture=False):
        """dims = (nh, nkv, d, rot, theta); w = dict(qn_w, kn_w).
        The caches are updated in place. Returns y (and q/k captures)."""
        nh, nkv, d, rot, theta = dims
        B = len(cu) - 1
        Ttot = int(cu[-1])
        y = np.empty((Ttot, nh * d), np.uint16)
        qf = np.empty((Ttot, nh * d), np.uint16) if capture else None
        kf = np.empty((Ttot, nkv * d), np.uint16) if capture else None
        self.lib.orc_attn_mixer(C.byref(_AttnDims(nh, nkv, d, rot, theta)),
                                u16(w["qn_w"]), u16(w["kn_w"]), _sz(B),
                                i32(cu), i32(pos0), u16(qg), u16(k), u16(v),
                                u16(kcache), u16(vcache), _sz(cache_stride),
                                u16(y), u16(qf), u16(kf), C.c_int(nthreads))
        return (y, qf, kf) if capture else y

    def attn_mixer_off(self, dims, w, cu, pos0, qg, k, v, kcache, vcache,
                       cache_off, nthreads=0, capture=False):
        """As attn_mixer with sequence s's caches at element offset
        cache_off[s] of the flat kcache/vcache arrays ([rows, nkv, d] from
        there). capture adds (qf, kf, attno): roped q, roped k and the
        attention output before the gate."""
        nh, nkv, d, rot, theta = dims
        B = len(cu) - 1
        Ttot = int(cu[-1])
        off = np.ascontiguousarray(cache_off, np.uint64)
        y = np.empty((Ttot, nh * d), np.uint16)
        qf = np.empty((Ttot, nh * d), np.uint16) if capture else None
        kf = np.empty((Ttot, nkv * d), np.uint16) if capture else None
        ao = np.empty((Ttot, nh * d), np.uint16) if capture else None
        self.lib.orc_attn_mixer_off(
            C.byref(_AttnDims(nh, nkv, d, rot, theta)), u16(w["qn_w"]),
            u16(w["kn_w"]), _sz(B), i32(cu), i32(pos0), u16(qg), u16(k),
            u16(v), u16(kcache), u16(vcache),
            off.ctypes.data_as(C.POINTER(_sz)), u16(y), u16(qf), u16(kf),
            u16(ao), C.c_int(nthreads))
        return (y, qf, kf, ao) if capture else y

    def attn_prep_off(self, dims, w, cu, pos0, qg, k, v, kcache, vcache,
                      cache_off, nthreads=0):
        """The mixer's norm / rope / append phase only; returns the roped
        q [Ttot, nh*d] (the caches are appended in place)."""
        nh, nkv, d, rot, theta = dims
        B = len(cu) - 1
        Ttot = int(cu[-1])
        off = np.ascontiguousarray(cache_off, np.uint64)
        qn = np.empty((Ttot, nh * d), np.uint16)
        self.lib.orc_attn_prep_off(
            C.byref(_AttnDims(nh, nkv, d, rot, theta)), u16(w["qn_w"]),
            u16(w["kn_w"]), _sz(B), i32(cu), i32(pos0), u16(qg), u16(k),
            u16(v), u16(kcache), u16(vcache),
            off.ctypes.data_as(C.POINTER(_sz)), u16(qn), None,
            C.c_int(nthreads))
        return qn


class Reference(_Ops):
    """The reference's own anchors built from /root/reference/c
    (oracle/ref_shim.c). Thread count comes from APUS_THREADS, read by the
    reference pool at its first parallel call."""

    def __init__(self):
        super().__init__(_load(REF_SO), "apus_")
        self.lib.ref_pool_threads.restype = C.c_int

    @staticmethod
    def available():
        return os.path.exists(REF_SO)

    def pool_threads(self):
        return self.lib.ref_pool_threads()

    def gdn_step_mt(self, S, q, k, v, g, beta, H, Dk, Dv):
        o = np.empty(H * Dv, np.float32)
        self.lib.apus_gdn_step_mt(f32(S), f32(q), f32(k), u16(v), f32(g),
                                  u16(beta), f32(o), _sz(H), _sz(Dk), _sz(Dv))
        return o

    def attn_gqa_mt(self, q, kc, vc, Tq, Tk, H, Hkv, D, scale):
        o = np.empty(Tq * H * D, np.uint16)
        self.lib.apus_attn_gqa_mt(u16(q), u16(kc), u16(vc), u16(o), _sz(Tq),
                                  _sz(Tk), _sz(H), _sz(Hkv), _sz(D),
                                  C.c_float(scale))
        return o

    def bf16_gemm(self, w, x, hot=True):
        """The reference's gemm: hot (threaded x86 path) or the scalar
        anchor, y [M,O]."""
        O, K = w.shape
        M = x.shape[0]
        y = np.empty((M, O), np.uint16)
        if hot:
            self.lib.ref_bf16_gemm_hot(u16(w), u16(x), u16(y), _sz(M), _sz(O), _sz(K))
        else:
            self.lib.apus_bf16_gemm_scalar(u16(w), u16(x), u16(y), _sz(M), _sz(O), _sz(K))
        return y

    def bf16_gemv(self, w, x):
        O, K = w.shape
        y = np.empty(O, np.uint16)
        self.lib.ref_bf16_gemv_hot(u16(w), u16(x), u16(y), _sz(O), _sz(K))
        return y

    def gdn_mixer(self, dims, w, cu, qkv, z, a, b, conv_state, S):
        hk, hv, dk, dv = dims
        B = len(cu) - 1
        y = np.empty((int(cu[-1]), hv * dv), np.uint16)
        self.lib.ref_gdn_mixer(_sz(hk), _sz(hv), _sz(dk), _sz(dv),
                               u16(w["conv_w"]), f32(w["A_log"]),
                               f32(w["dt_bias"]), u16(w["onorm_w"]), _sz(B),
                               i32(cu), u16(qkv), u16(z), u16(a), u16(b),
                               u16(conv_state), f32(S), u16(y))
        return y

    def attn_mixer(self, dims, w, cu, pos0, qg, k, v, kcache, vcache,
                   cache_stride):
        nh, nkv, d, rot, theta = dims
        B = len(cu) - 1
        y = np.empty((int(cu[-1]), nh * d), np.uint16)
        self.lib.ref_attn_mixer(_sz(nh), _sz(nkv), _sz(d), _sz(rot),
                                C.c_double(theta), u16(w["qn_w"]),
                                u16(w["kn_w"]), _sz(B), i32(cu), i32(pos0),
                                u16(qg), u16(k), u16(v), u16(kcache),
                                u16(vcache), _sz(cache_stride), u16(y))
        return y
