"""Benchmark of the apus-qwen attention hot path on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--only c0,c0b,c1,...]
                [--no-cpu]

A "step" is one pass of a mixer (the hot path between a layer's input
projections and its output projection) over one batch of synthetic inputs
already resident in HBM. The headline line is BASELINE config 4, the largest
single-GPU configuration: one hybrid decode block (3 Gated DeltaNet layers +
1 gated-GQA layer) over 128 sequences verifying 1..4 tokens each at
log-normal cached contexts, reported as verified tokens per second through
the block. Every configuration is measured in the same run and reported
under "configs" with its own roofline fraction against MI355X's published
peaks (HBM 8 TB/s, dense bf16 MFMA 2.5 PFLOP/s):
  c0   config 0   GDN decode, batch 1
  c0b  config 0'  GDN decode, batch 64 (HBM-bound decode)
  c1   config 1   GDN prefill T=4096
  c2   config 2   gated-GQA decode, 64 sequences x 32K-token bf16 KV cache
  c3   config 3   gated-GQA causal prefill, T=8192 (cache fill + attention)
  c4   config 4   hybrid decode block, 3 GDN + 1 GQA layers, 128 sequences
                  (headline)
  c4p  config 4   the same block with every layer's projections (layer
                  entry points: one input-projection launch, mixer, output
                  projection)
  p1, p64, p4096  the GDN input projection (2048 -> 12352) beside the path:
                  1 token (reference-order kernel, bitwise), 64 and 4096
                  tokens (the hand-written MFMA GEMM)
Input buffer sets rotate (at least 4 where the inputs are smaller than the
256 MB Infinity Cache) so repeated reads come from HBM.

The CPU leg (skipped with --no-cpu) does two things per configuration:
  * parity: one more GPU step on buffer set 0, whose inputs (and prior
    state and caches) are copied back and run through the CPU oracle
    (oracle/, the C restatement of the reference anchors); the line reports
    the measured worst case (normwise relative error, bf16 ulps, fraction of
    bit-identical outputs, state error) against the north star's bars;
  * cpu_baseline: the repo's C restatement of the reference's scalar
    anchors (oracle/apus_oracle.c, pinned bitwise to the reference's own
    c/gdn.h / c/attn.h by the CPU tests; kind "port") timed on the host
    cores on a bounded sample of each configuration, at min(32, cores)
    threads (the reference pool's lane cap) and at all the cores this
    process may use.
"""
import argparse
import json
import os
import platform
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "apus-qwen3.6-35b-a3b_amd")
for p in (PKG, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK = 8.0e12            # B/s, MI355X HBM3E
BF16_PEAK = 2.5e15           # flop/s dense bf16 MFMA
FP32_PEAK = 157.3e12         # flop/s dense fp32 MFMA

GDN = (16, 32, 128, 128)
HK, HV, DK, DV = GDN
CD = 2 * HK * DK + HV * DV   # conv_dim 8192
VD = HV * DV                 # value_dim 4096


# ---------------------------------------------------------------- helpers
def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gdn_seq_bytes(ntok):
    """Algorithmic HBM bytes of one GDN sequence over ntok tokens:
    S read+write, conv state read+write, per token qkv, z, a, b in and y
    out (state touched once however many tokens)."""
    state = HV * DK * DV * 4 * 2 + CD * 3 * 2 * 2
    per_tok = CD * 2 + VD * 2 + HV * 2 * 2 + VD * 2
    return state + ntok * per_tok


GDN_WEIGHT_BYTES = CD * 4 * 2 + HV * 4 * 2 + DV * 2


class Dev:
    """Device buffers for one GDN workload with `nsets` rotating sets."""

    def __init__(self, torch, B, T_per_seq, nsets, seed, zero_state):
        import apus_hip
        self.torch = torch
        dev = torch.device("cuda")
        g = torch.Generator(device=dev)
        g.manual_seed(seed)

        def bf(shape, std=1.0, mean=0.0):
            x = torch.randn(shape, generator=g, device=dev, dtype=torch.float32) * std + mean
            return x.to(torch.bfloat16).view(torch.int16)

        self.w = dict(conv_w=bf((CD, 4), 0.1),
                      A_log=torch.rand(HV, generator=g, device=dev) * 2.7,
                      dt_bias=torch.ones(HV, device=dev),
                      onorm_w=bf((DV,), 0.1, 1.0))
        self.layer = apus_hip.gdn_layer(GDN, self.w)
        T = B * T_per_seq
        self.cu = np.arange(B + 1, dtype=np.int32) * T_per_seq
        self.sets = []
        for _ in range(nsets):
            s = dict(qkv=bf((T, CD)), z=bf((T, VD)), a=bf((T, HV)), b=bf((T, HV)),
                     y=torch.empty((T, VD), dtype=torch.int16, device=dev))
            if zero_state:
                s["conv"] = torch.zeros((B, CD * 3), dtype=torch.int16, device=dev)
                s["S"] = torch.zeros((B, HV, DK, DV), dtype=torch.float32, device=dev)
            else:
                s["conv"] = bf((B, CD * 3))
                s["S"] = torch.randn((B, HV, DK, DV), generator=g, device=dev) * 0.02
            self.sets.append(s)
        self.zero_state = zero_state


def time_steps(torch, fn, steps, warmup, nsets, kernels=()):
    """Run warmup then `steps` timed steps; return (total_s, per-step event
    times in s, {kernel: average launch ms}). Each step uses buffer set
    i % nsets. The wall-clock pass runs the steps back to back with nothing
    else enqueued (an event record between steps adds its own gap on the
    GPU, a visible share of a short step). A second pass records HIP events
    around each step, a third around each launch of the named kernels on
    the library's stream (apus_hip_timing_*). The collector runs before and
    stays off during each pass: a generation-2 collection over the
    process's objects takes 15-40 ms, enough to drain the launch queue in
    the middle of a timed pass."""
    import gc
    import apus_hip
    for i in range(warmup):
        fn(i % nsets)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    gc.collect()
    gc.disable()
    try:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            fn(i % nsets)
        torch.cuda.synchronize()
        total = time.perf_counter() - t0
        for i in range(steps):
            ev[i][0].record()
            fn(i % nsets)
            ev[i][1].record()
        torch.cuda.synchronize()
    finally:
        gc.enable()
    per = [a.elapsed_time(b) * 1e-3 for a, b in ev]
    kt = {}
    if kernels:
        gc.collect()
        gc.disable()
        apus_hip.timing_enable(True)
        try:
            for i in range(steps):
                fn(i % nsets)
        finally:
            gc.enable()
        for k in kernels:
            ms, n = apus_hip.timing_get(k)
            if n:
                kt[k] = ms / n
        apus_hip.timing_enable(False)
    return total, per, kt


def measured_traffic(workload, kernel):
    """HBM bytes per launch of `kernel` in `workload` from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes (profiles/hbm_traffic.json,
    scaled by a 1 GiB copy), or None when not profiled."""
    try:
        with open(os.path.join(ROOT, "profiles", "hbm_traffic.json")) as f:
            t = json.load(f)
        return t[f"{workload}/{kernel}"]["bytes"]
    except (OSError, KeyError, ValueError):
        return None


def kernel_roofline(kt, table, workload):
    """Roofline of the dominant kernel (the longest average launch): table
    maps kernel name to (bound, algorithmic units per launch, peak per
    second[, note]); achieved = units / that kernel's average launch time
    (HIP events on the library stream). Peaks are MI355X's published ones.
    traffic is the kernel's HBM bytes per launch from the committed
    rocprofv3 counter passes named in traffic_source (counters cannot be
    read inside this process)."""
    name = max((k for k in table if k in kt), key=lambda k: kt[k])
    bound, units, peak = table[name][:3]
    sec = kt[name] * 1e-3
    traffic = measured_traffic(workload, name)
    r = dict(kernel=name, bound=bound, launch_ms=kt[name], per_launch=units)
    if bound == "mfma":
        r.update(achieved=units / sec / 1e12, peak=peak / 1e12, unit="TFLOP/s")
    else:
        r.update(achieved=units / sec / 1e9, peak=peak / 1e9, unit="GB/s")
    r["frac"] = units / sec / peak
    r["traffic"] = traffic
    r["traffic_source"] = ("profiles/hbm_traffic.json: rocprofv3 --pmc FETCH_SIZE then WRITE_SIZE "
                           "passes of this workload, scaled by a 1 GiB copy" if traffic else None)
    if len(table[name]) > 3:
        r.update(table[name][3])
    return r


# ---------------------------------------------------------------- parity
def _h16(t):
    return t.cpu().numpy().view(np.uint16)


def _bf16_f64(codes):
    return (np.asarray(codes, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def _ulps(a, b):
    o = lambda c: np.where(c & 0x8000, 0x8000 - c, c)
    return np.abs(o(np.asarray(a, np.int64)) - o(np.asarray(b, np.int64)))


def bf16_cmp(c, r):
    """Measured worst case of bf16 outputs c against the oracle's r:
    normwise relative error, fraction of bit-identical codes, and the
    largest bf16 ulp distance among elements whose difference exceeds 1e-3
    of the tensor's rms (elements small through cancellation excluded)."""
    c, r = np.asarray(c).ravel(), np.asarray(r).ravel()
    cf, rf = _bf16_f64(c), _bf16_f64(r)
    nr = np.linalg.norm(rf)
    ud = _ulps(c, r)
    far = np.abs(cf - rf) > 1e-3 * np.sqrt(np.mean(rf * rf))
    return dict(rel=float(np.linalg.norm(cf - rf) / nr) if nr else 0.0,
                exact=float(np.mean(ud == 0)), max_ulp=int(ud[far].max()) if far.any() else 0,
                n=int(c.size))


def _esc_judge(c, r, esc, ulps=2):
    """The attention tolerance class per element (tests/numerics.py
    assert_bf16_esc): elements more than `ulps` bf16 ulps from the oracle
    must lie within 2e-3 (|r| + esc), esc the sum of |P_j V_j| with the
    rounding-flip allowance (tests/attn_util.py). max_ulp above counts
    elements small through cancellation, whose ulps are not a measure of
    error; esc_max is the bar's own quantity."""
    c, r = np.asarray(c).ravel(), np.asarray(r).ravel()
    cf, rf = _bf16_f64(c), _bf16_f64(r)
    ratio = np.abs(cf - rf) / (np.abs(rf) + np.asarray(esc, np.float64).ravel() + 1e-30)
    judged = _ulps(c, r) > ulps
    return dict(esc_max=float(ratio[judged].max()) if judged.any() else 0.0,
                esc_max_all=float(ratio.max()) if ratio.size else 0.0)


def state_rel(c, r):
    den = float(np.max(np.abs(r)))
    return float(np.max(np.abs(c.astype(np.float64) - r))) / den if den else 0.0


class CpuLeg:
    """The oracle as the checker of the GPU results (never measured)."""

    def __init__(self):
        import oracle
        self.orc = oracle.Oracle()
        self.nt = _avail_cores()

    def gdn(self, torch, layer_w, cu, tok, conv0, S0, y, conv1, S1, prefill=False):
        """One GDN mixer step: host inputs tok (device tensors), prior state
        (host), GPU results (device); returns the comparison."""
        import apus_hip
        w = {k: (_h16(v) if v.dtype == torch.int16 else v.cpu().numpy()) for k, v in layer_w.items()}
        t = {k: _h16(v) for k, v in tok.items()}
        c_o, S_o = conv0.copy(), S0.copy()
        y_o = self.orc.gdn_mixer(GDN, w, np.asarray(cu, np.int32), t["qkv"], t["z"], t["a"],
                                 t["b"], c_o, S_o, nthreads=self.nt)
        Sr = torch.empty_like(S1)
        apus_hip.gdn_state_unpack(S1, Sr)
        torch.cuda.synchronize()
        r = bf16_cmp(_h16(y), y_o)
        r["state_rel"] = state_rel(Sr.cpu().numpy(), S_o)
        r["conv_exact"] = bool(np.array_equal(_h16(conv1), c_o))
        bar_ulp = 4 if prefill else 1
        r["pass"] = bool(r["rel"] <= 2e-3 and r["max_ulp"] <= bar_ulp and r["state_rel"] <= 1e-4
                         and r["conv_exact"])
        return r

    def attn(self, torch, w, cu, pos0, tok, caches, y, rows=None):
        """GQA mixer: caches = list of (K, V) host reference-layout arrays per
        sequence as the GPU left them (the appended rows included), which the
        oracle re-appends bit-identically from the same inputs; rows (optional)
        restricts the comparison to sampled query rows of a one-sequence
        prefill, recomputed by the oracle's ordered GQA rows."""
        wh = {k: _h16(v) for k, v in w.items()}
        t = {k: _h16(v) for k, v in tok.items()}
        B = len(cu) - 1
        nrow = [int(K.shape[0]) for K, _ in caches]
        off = np.concatenate([[0], np.cumsum(np.asarray(nrow, np.int64) * NKV * AD)])
        kk = np.concatenate([K.reshape(-1) for K, _ in caches])
        vv = np.concatenate([V.reshape(-1) for _, V in caches])
        kg, vg = kk.copy(), vv.copy()
        yh = _h16(y)
        from attn_util import attn_esc_rows
        if rows is None:
            y_o, qf, _, _ = self.orc.attn_mixer_off(ATTN, wh, np.asarray(cu, np.int32),
                                                    np.asarray(pos0, np.int32), t["qg"], t["k"],
                                                    t["v"], kk, vv, off[:-1], nthreads=self.nt,
                                                    capture=True)
            r = bf16_cmp(yh, y_o)
            esc = np.concatenate([
                attn_esc_rows(qf[cu[s]:cu[s + 1]], kk[off[s]:off[s + 1]].reshape(-1, NKV, AD),
                              vv[off[s]:off[s + 1]].reshape(-1, NKV, AD),
                              int(pos0[s]) + np.arange(cu[s + 1] - cu[s]), NH, NKV, AD)
                for s in range(B) if cu[s + 1] > cu[s]])
            r.update(_esc_judge(yh, y_o, esc))
        else:
            qn = self.orc.attn_prep_off(ATTN, wh, np.asarray(cu, np.int32),
                                        np.asarray(pos0, np.int32), t["qg"], t["k"], t["v"],
                                        kk, vv, off[:-1], nthreads=self.nt)
            Tn = int(cu[-1])
            K, V = kk.reshape(Tn, NKV, AD), vv.reshape(Tn, NKV, AD)
            gate = t["qg"].reshape(Tn, NH, 2 * AD)[:, :, AD:]
            got, want = [], []
            for r0, r1 in rows:
                ao = self.orc.attn_gqa_mt(np.ascontiguousarray(qn[r0:r1]), np.ascontiguousarray(K[:r1]),
                                          np.ascontiguousarray(V[:r1]), r1 - r0, r1, NH, NKV, AD,
                                          np.float32(1.0 / 16.0), nthreads=self.nt)
                want.append(self.orc.attn_outgate(ao, np.ascontiguousarray(gate[r0:r1]).reshape(-1)))
                got.append(yh[r0:r1].reshape(-1))
            r = bf16_cmp(np.concatenate(got), np.concatenate(want))
            r["rows"] = [list(x) for x in rows]
            esc = np.concatenate([attn_esc_rows(qn[r0:r1], K, V, np.arange(r0, r1), NH, NKV, AD)
                                  for r0, r1 in rows])
            r.update(_esc_judge(np.concatenate(got), np.concatenate(want), esc))
        r["cache_exact"] = bool(np.array_equal(kk, kg) and np.array_equal(vv, vg))
        r["pass"] = bool(r["rel"] <= 2e-3 and r["esc_max"] <= 2e-3 and r["cache_exact"])
        return r


def _host_caches(torch, kc, vc, max_seq, nrows):
    """Reference-layout host copies of the first nrows[s] positions of each
    sequence's device cache."""
    import apus_hip
    out = []
    for s, n in enumerate(nrows):
        rk = torch.empty((int(n), NKV, AD), dtype=torch.int16, device="cuda")
        rv = torch.empty_like(rk)
        apus_hip.attn_cache_unpack(kc[s], vc[s], int(n), NKV, AD, max_seq, rk, rv)
        torch.cuda.synchronize()
        out.append((_h16(rk), _h16(rv)))
    return out


def _gdn_state_host(torch, S):
    import apus_hip
    Sr = torch.empty_like(S)
    apus_hip.gdn_state_unpack(S, Sr)
    torch.cuda.synchronize()
    return Sr.cpu().numpy()


# ---------------------------------------------------------------- workloads
def bench_gdn_decode(torch, B, steps, warmup, seed, leg=None):
    """Config 0 / 0': one decode token per sequence, prior state."""
    import apus_hip
    nsets = 4 if B > 1 else 8
    d = Dev(torch, B, 1, nsets, seed, zero_state=False)

    # each set's call prepared once (apus_hip.BoundCall): a decode step is
    # one launch, so per-call argument conversion would be a visible share
    # of the wall time
    calls = [apus_hip.gdn_decode_bound(d.layer, d.cu, s["qkv"], s["z"], s["a"], s["b"], s["conv"],
                                       s["S"], s["y"]) for s in d.sets]

    def step(i):
        calls[i]()

    bytes_ = B * gdn_seq_bytes(1) + GDN_WEIGHT_BYTES
    table = {"k_gdn_decode": ("hbm", bytes_, HBM_PEAK)}
    total, per, kt = time_steps(torch, step, steps, warmup, nsets, table)
    st = float(np.mean(per))
    wl = f"gdn_decode_b{B}"
    r = dict(workload=wl, tokens_per_step=B, ms_per_step=total / steps * 1e3,
             step_event_ms=st * 1e3, step_event_median_ms=float(np.median(per)) * 1e3, kernels_ms=kt, alg_bytes=bytes_,
             tok_s=B * steps / total, roofline=kernel_roofline(kt, table, wl))
    if leg:
        s = d.sets[0]
        conv0, S0 = _h16(s["conv"]), _gdn_state_host(torch, s["S"])
        step(0)
        r["parity"] = leg.gdn(torch, d.w, d.cu, {k: s[k] for k in ("qkv", "z", "a", "b")},
                              conv0, S0, s["y"], s["conv"], s["S"])
    return r


def bench_gdn_prefill(torch, T, steps, warmup, seed, leg=None):
    """Config 1: one sequence of T tokens. The first step of each buffer set
    starts from a zero state; later ones continue from the state the set's
    previous step left, which the kernels process identically (the work is
    data-independent), so no state reset sits in the timed region."""
    import apus_hip
    nsets = 4
    d = Dev(torch, 1, T, nsets, seed, zero_state=True)

    def step(i):
        s = d.sets[i]
        apus_hip.gdn_prefill(d.layer, d.cu, s["qkv"], s["z"], s["a"], s["b"], s["conv"], s["S"], s["y"])

    bytes_ = gdn_seq_bytes(T) + GDN_WEIGHT_BYTES
    flops = gdn_prefill_flops(T)
    nu = (T // 64) * HV                       # (chunk, v-head) units
    # WY and the scan multiply on the bf16 MFMA; fp32 operands are split
    # (hi + lo, a product against another split operand is three MFMAs,
    # against exact bf16 codes two). frac is against the published bf16
    # peak, split_roof_frac against the share of it the executed MFMA work
    # leaves for the algorithm's flops (SCAN/WY_EXEC_PER_UNIT below)
    table = {"k_gdn_chunk_scan": ("mfma", nu * SCAN_FLOPS_PER_UNIT, BF16_PEAK,
                                  {"split_roof_tflops": BF16_PEAK * SCAN_FLOPS_PER_UNIT
                                   / SCAN_EXEC_PER_UNIT / 1e12}),
             "k_gdn_chunk_wy": ("mfma", nu * WY_FLOPS_PER_UNIT, BF16_PEAK,
                                {"split_roof_tflops": BF16_PEAK * WY_FLOPS_PER_UNIT
                                 / WY_EXEC_PER_UNIT / 1e12}),
             "k_gdn_post": ("hbm", gdn_post_bytes(T), HBM_PEAK)}
    total, per, kt = time_steps(torch, step, steps, warmup, nsets, table)
    st = float(np.mean(per))
    wl = f"gdn_prefill_t{T}"
    roof = kernel_roofline(kt, table, wl)
    if "split_roof_tflops" in roof:
        roof["split_roof_frac"] = roof["achieved"] / roof["split_roof_tflops"]
    r = dict(workload=wl, tokens_per_step=T, ms_per_step=total / steps * 1e3,
             step_event_ms=st * 1e3, step_event_median_ms=float(np.median(per)) * 1e3, kernels_ms=kt, alg_bytes=bytes_, alg_flops=flops,
             tok_s=T * steps / total, layer_hbm_frac=bytes_ / st / HBM_PEAK,
             layer_tflops=flops / st / 1e12, layer_mfma_frac=flops / st / BF16_PEAK,
             roofline=roof)
    if leg:
        s = d.sets[0]
        conv0, S0 = _h16(s["conv"]), _gdn_state_host(torch, s["S"])
        step(0)
        r["parity"] = leg.gdn(torch, d.w, d.cu, {k: s[k] for k in ("qkv", "z", "a", "b")},
                              conv0, S0, s["y"], s["conv"], s["S"], prefill=True)
    return r


# Algorithmic flops per (chunk of 64, v-head) of the two chunk kernels:
# the scan does W S0, Q S0, K^T D (64x128x128 each) and A D (64x64x128);
# the WY build does K K^T, Q K^T (64x64x128, on the q/k codes shared by the
# two v-heads of a K head, so half of each per v-head unit) and the two
# 64x64x128 triangular applications giving U and W, plus the triangular
# solve.
SCAN_FLOPS_PER_UNIT = 3 * 2 * 64 * 128 * 128 + 2 * 64 * 64 * 128
WY_FLOPS_PER_UNIT = 3 * 2 * 64 * 64 * 128 + (2 * 64 ** 3) // 3
# MFMA flops the kernels execute for them: the scan's W S0 and A D take
# three MFMAs per product (both operands split), Q S0 and K^T D two (q, k
# as exact codes); WY's K K^T and Q K^T one (codes), T R two, and the
# 32x32 off-diagonal block of T two split products
SCAN_EXEC_PER_UNIT = 3 * 2 * 64 * 128 * 128 + 2 * 2 * 2 * 64 * 128 * 128 + 3 * 2 * 64 * 64 * 128
WY_EXEC_PER_UNIT = 2 * 2 * 64 * 64 * 128 + 2 * 2 * 2 * 64 * 64 * 128 + 3 * 2 * 2 * 32 ** 3


def gdn_post_bytes(T):
    """k_gdn_post interface bytes: rnd(o) and z in, y out; conv state
    rewritten from the last three qkv rows."""
    return T * VD * 2 * 3 + CD * 3 * 2 * 2 + 3 * CD * 2


def gdn_prefill_flops(T, C=64):
    """WY-form flops per (chunk, head): 5 matmuls of 64x64x128-class
    (2*64*64*128 = 1,048,576 each), 3 of 64x128x128 (2,097,152 each) and
    the triangular solve (~64^3*2/3 = 174,763); x chunks x 32 heads."""
    per = 5 * 2 * C * C * DK + 3 * 2 * C * DK * DV + (2 * C ** 3) // 3
    return per * (T // C) * HV


ATTN = (16, 2, 256, 64, 1e7)
NH, NKV, AD = 16, 2, 256
HID = 2048                  # hidden size (the projections' K / output)


def attn_decode_bytes(ctx, tq=1):
    """Algorithmic HBM bytes of one sequence's decode step: the K and V
    cache rows read (ctx keys x nkv x d x 2 B each), the new q|gate, k, v
    read, the appended k, v written, and the gated output written."""
    kv = ctx * NKV * AD * 2 * 2
    per_tok = NH * 2 * AD * 2 + NKV * AD * 2 * 2 + NKV * AD * 2 * 2 + NH * AD * 2
    return kv + tq * per_tok


def _bf_gen(torch, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)

    def bf(shape, std=1.0, mean=0.0):
        x = torch.randn(shape, generator=g, device="cuda", dtype=torch.float32) * std + mean
        return x.to(torch.bfloat16).view(torch.int16)
    return g, bf


def bench_attn_decode(torch, B, ctx, steps, warmup, seed, leg=None):
    """Config 2: B sequences, each with ctx-1 cached tokens plus one new
    token (so the new token attends ctx keys). The 4 GiB of caches dwarf
    the Infinity Cache; two small q/k/v sets alternate."""
    import apus_hip
    g, bf = _bf_gen(torch, seed)
    w = dict(qn_w=bf((AD,), 0.1), kn_w=bf((AD,), 0.1))
    layer = apus_hip.attn_layer(ATTN, w)
    max_seq = ctx
    kc = bf((B, NKV, max_seq, AD))
    vc = bf((B, NKV, max_seq // 32, AD, 32))
    nsets = 2
    sets = [dict(qg=bf((B, NH, 2 * AD)), k=bf((B, NKV, AD)), v=bf((B, NKV, AD)),
                 y=torch.empty((B, NH * AD), dtype=torch.int16, device="cuda")) for _ in range(nsets)]
    cu = np.arange(B + 1, dtype=np.int32)
    pos0 = np.full(B, ctx - 1, np.int32)

    def step(i):
        s = sets[i]
        apus_hip.attn_decode(layer, cu, pos0, s["qg"], s["k"], s["v"], kc, vc, max_seq, s["y"])

    bytes_ = B * attn_decode_bytes(ctx) + 2 * AD * 2
    flops = B * NH * 4 * AD * ctx
    kbytes = B * ctx * NKV * AD * 2           # one of the K / V caches
    table = {"k_attn_scores": ("hbm", kbytes, HBM_PEAK), "k_attn_pv": ("hbm", kbytes, HBM_PEAK),
             "k_attn_prep": ("hbm", B * (NH * AD * 2 * 2 + 2 * NKV * AD * 2 * 2), HBM_PEAK),
             "k_attn_combine": ("hbm", B * NH * AD * 2 * 2, HBM_PEAK)}
    total, per, kt = time_steps(torch, step, steps, warmup, nsets, table)
    st = float(np.mean(per))
    wl = f"attn_decode_b{B}_ctx{ctx}"
    r = dict(workload=wl, tokens_per_step=B, ms_per_step=total / steps * 1e3,
             step_event_ms=st * 1e3, step_event_median_ms=float(np.median(per)) * 1e3, kernels_ms=kt, alg_bytes=bytes_, alg_flops=flops,
             tok_s=B * steps / total, layer_hbm_gbs=bytes_ / st / 1e9,
             layer_hbm_frac=bytes_ / st / HBM_PEAK, roofline=kernel_roofline(kt, table, wl))
    if leg:
        s = sets[0]
        step(0)
        pick = [0, 21, 42, 63][: min(4, B)]          # sampled sequences
        caches = _host_caches(torch, kc[pick], vc[pick], max_seq, [ctx] * len(pick))
        sub = lambda t: t[pick]
        r["parity"] = leg.attn(torch, w, np.arange(len(pick) + 1, dtype=np.int32), pos0[pick],
                               {k: sub(s[k]) for k in ("qg", "k", "v")}, caches, sub(s["y"]))
        r["parity"]["sample"] = f"sequences {pick} of {B}"
    return r


def attn_prefill_flops(T):
    """Causal GQA prefill, algorithmic: q.k and P.V over the keys each row
    sees (16 heads x 256 dims x 2 flop x 2 matmuls x T(T+1)/2 rows-keys)."""
    return NH * 4 * AD * (T * (T + 1) // 2)


PREFILL_SAMPLE_ROWS = ((0, 64), (2047, 2111), (4096, 4160), (8128, 8192))


def bench_attn_prefill(torch, T, steps, warmup, seed, leg=None):
    """Config 3: one sequence, T new tokens from position 0: norm, RoPE,
    cache fill and causal attention with the output gate."""
    import apus_hip
    g, bf = _bf_gen(torch, seed)
    w = dict(qn_w=bf((AD,), 0.1), kn_w=bf((AD,), 0.1))
    layer = apus_hip.attn_layer(ATTN, w)
    nsets = 4
    sets = [dict(qg=bf((T, NH, 2 * AD)), k=bf((T, NKV, AD)), v=bf((T, NKV, AD)),
                 kc=torch.empty((1, NKV, T, AD), dtype=torch.int16, device="cuda"),
                 vc=torch.empty((1, NKV, T // 32, AD, 32), dtype=torch.int16, device="cuda"),
                 y=torch.empty((T, NH * AD), dtype=torch.int16, device="cuda")) for _ in range(nsets)]
    cu = np.array([0, T], np.int32)
    pos0 = np.zeros(1, np.int32)

    def step(i):
        s = sets[i]
        apus_hip.attn_prefill(layer, cu, pos0, s["qg"], s["k"], s["v"], s["kc"], s["vc"], T, s["y"])

    flops = attn_prefill_flops(T)
    bytes_ = T * (NH * 2 * AD * 2 + 2 * NKV * AD * 2 + 2 * NKV * AD * 2 + NH * AD * 2)
    table = {"k_attn_fa": ("mfma", flops, BF16_PEAK),
             # q and k rows read and written (normed, roped), v rows appended
             "k_attn_prep": ("hbm", T * (NH * AD * 2 * 2 + 2 * NKV * AD * 2 * 2), HBM_PEAK)}
    total, per, kt = time_steps(torch, step, steps, warmup, nsets, table)
    st = float(np.mean(per))
    wl = f"attn_prefill_t{T}"
    r = dict(workload=wl, tokens_per_step=T, ms_per_step=total / steps * 1e3,
             step_event_ms=st * 1e3, step_event_median_ms=float(np.median(per)) * 1e3, kernels_ms=kt, alg_bytes=bytes_, alg_flops=flops,
             tok_s=T * steps / total, layer_tflops=flops / st / 1e12,
             layer_mfma_frac=flops / st / BF16_PEAK, roofline=kernel_roofline(kt, table, wl))
    if leg:
        s = sets[0]
        step(0)
        caches = _host_caches(torch, s["kc"], s["vc"], T, [T])
        rows = [x for x in PREFILL_SAMPLE_ROWS if x[1] <= T]
        r["parity"] = leg.attn(torch, w, cu, pos0, {k: s[k] for k in ("qg", "k", "v")}, caches,
                               s["y"], rows=rows)
        r["parity"]["sample"] = "all 16 heads of the query rows listed; the whole cache fill"
    return r


def bench_mixed_block(torch, B, steps, warmup, seed, leg=None, proj=False):
    """Config 4: one hybrid decode block in the model's 3:1 ratio -- three
    Gated DeltaNet layers (each with its own weights, conv state and
    recurrent state per sequence) and one gated-GQA layer (a bf16 KV cache
    per sequence) -- over B sequences that each verify 1..4 tokens at a
    log-normal cached context. value = verified tokens per second through
    the block. The states live as a serving engine keeps them: the GDN
    states in a slot pool (apus_hip_gdn_pool_*, slots in shuffled order)
    and the KV cache in 32-position blocks of a paged pool sized to the
    contexts (apus_hip_kv_pool_*; blocks handed out interleaved across
    sequences, no per-sequence maximum reserved). The recurrent states
    (3 x 256 MB) and caches (GBs) exceed the Infinity Cache, so one input
    set is used."""
    import apus_hip
    import synth
    g, bf = _bf_gen(torch, seed)
    rng = np.random.default_rng(seed)
    ctx, k = synth.mixed_block_shape(B, seed)
    cu = np.concatenate([[0], np.cumsum(k)]).astype(np.int32)
    T = int(cu[-1])
    gpool = apus_hip.GdnPool(3, GDN, B + 8)
    opened = [gpool.open() for _ in range(B + 8)]
    slots = [opened[i] for i in rng.permutation(B + 8)[:B]]
    gdn = []
    for li in range(3):
        w = dict(conv_w=bf((CD, 4), 0.1), A_log=torch.rand(HV, generator=g, device="cuda") * 2.7,
                 dt_bias=torch.ones(HV, device="cuda"), onorm_w=bf((DV,), 0.1, 1.0))
        conv, S = gpool.state(li)
        gdn.append(dict(layer=apus_hip.gdn_layer(GDN, w), w=w, qkv=bf((T, CD)), z=bf((T, VD)),
                        a=bf((T, HV)), b=bf((T, HV)), conv=conv, S=S,
                        y=torch.empty((T, VD), dtype=torch.int16, device="cuda")))
        for sl in slots:                    # prior state: conv ~ N(0,1), S ~ N(0, 0.02)
            gpool.load_state(li, sl, bf((CD * 3,)),
                             torch.randn((HV, DK, DV), generator=g, device="cuda") * 0.02)
    aw = dict(qn_w=bf((AD,), 0.1), kn_w=bf((AD,), 0.1))
    alayer = apus_hip.attn_layer(ATTN, aw)
    nblk = -(-(ctx + k) // 32)
    kpool = apus_hip.KvPool(1, NKV, AD, int(nblk.sum()), B, int(nblk.max()))
    rows = [kpool.open() for _ in range(B)]
    have = np.zeros(B, np.int64)
    while (have < nblk).any():                  # blocks interleaved across sequences
        for s in rng.permutation(B):
            if have[s] < nblk[s]:
                have[s] += 1
                kpool.reserve(rows[s], int(have[s]) * 32)
    kv = kpool.cache(0)

    # caches filled with N(0, 1) bf16 values (config 2's distribution)
    for s in range(B):
        apus_hip.attn_cache_pack_paged(bf((int(ctx[s]), NKV, AD)), bf((int(ctx[s]), NKV, AD)),
                                       int(ctx[s]), NKV, AD, kv, rows[s])
    att = dict(qg=bf((T, NH, 2 * AD)), k=bf((T, NKV, AD)), v=bf((T, NKV, AD)),
               y=torch.empty((T, NH * AD), dtype=torch.int16, device="cuda"))
    if proj:
        # each layer's projections (c/layer.h:133-157 layouts), its normed
        # input ln1 and its projected output ao
        sH = HID ** -0.5
        for L in gdn:
            L["pw"] = dict(w_qkv=bf((CD, HID), sH), w_z=bf((VD, HID), sH), w_b=bf((HV, HID), sH),
                           w_a=bf((HV, HID), sH), w_out=bf((HID, VD), VD ** -0.5))
            L["proj"] = apus_hip.gdn_proj(HID, L["pw"])
            L["ln1"] = bf((T, HID))
            L["ao"] = torch.empty((T, HID), dtype=torch.int16, device="cuda")
        att["pw"] = dict(wq=bf((NH * 2 * AD, HID), sH), wk=bf((NKV * AD, HID), sH),
                         wv=bf((NKV * AD, HID), sH), wo=bf((HID, NH * AD), (NH * AD) ** -0.5))
        att["proj"] = apus_hip.attn_proj(HID, att["pw"])
        att["ln1"] = bf((T, HID))
        att["ao"] = torch.empty((T, HID), dtype=torch.int16, device="cuda")
    torch.cuda.synchronize()

    def step(i):
        if proj:
            for L in gdn:
                apus_hip.gdn_layer_decode_slots(L["layer"], L["proj"], slots, slots, cu, L["ln1"],
                                                L["conv"], L["S"], L["ao"])
            apus_hip.attn_layer_decode_paged(alayer, att["proj"], rows, cu, ctx, att["ln1"], kv,
                                             att["ao"])
            return
        for L in gdn:
            apus_hip.gdn_decode_slots(L["layer"], slots, slots, cu, L["qkv"], L["z"], L["a"],
                                      L["b"], L["conv"], L["S"], L["y"])
        apus_hip.attn_decode_paged(alayer, rows, cu, ctx, att["qg"], att["k"], att["v"], kv,
                                   att["y"])

    gdn_bytes = sum(gdn_seq_bytes(int(x)) for x in k) + GDN_WEIGHT_BYTES
    attn_bytes = sum(attn_decode_bytes(int(c) + int(x), int(x)) for c, x in zip(ctx, k)) + 2 * AD * 2
    bytes_ = 3 * gdn_bytes + attn_bytes
    kv1 = int(sum((int(c) + int(x)) * NKV * AD * 2 for c, x in zip(ctx, k)))   # one of K / V
    table = {"k_gdn_decode": ("hbm", gdn_bytes, HBM_PEAK),
             "k_attn_scores": ("hbm", kv1, HBM_PEAK), "k_attn_pv": ("hbm", kv1, HBM_PEAK),
             "k_attn_prep": ("hbm", T * (NH * AD * 2 * 2 + 2 * NKV * AD * 2 * 2), HBM_PEAK),
             "k_attn_combine": ("hbm", T * NH * AD * 2 * 2, HBM_PEAK)}
    if proj:
        # the projections' compulsory bytes: every weight once, ln1 in and
        # ao out per layer (the projection outputs the mixers read are
        # intermediates); the mixers' own terms already count their in/out
        # activations, which here are those intermediates
        w_gdn = ((CD + VD + 2 * HV) * HID + HID * VD) * 2
        w_att = ((NH * 2 * AD + 2 * NKV * AD) * HID + HID * NH * AD) * 2
        bytes_ += 3 * w_gdn + w_att + 4 * 2 * T * HID * 2
        flops_in = 2 * T * HID * (3 * (CD + VD + 2 * HV) + NH * 2 * AD + 2 * NKV * AD)
        flops_out = 2 * T * HID * (3 * VD + NH * AD)
        table["k_gemm_tile_in"] = ("hbm", (3 * (CD + VD + 2 * HV) + NH * 2 * AD + 2 * NKV * AD)
                                   * HID * 2 // 4 + T * HID * 2, HBM_PEAK)
        table["k_gemm_tile_out"] = ("hbm", (3 * HID * VD + HID * NH * AD) * 2 // 4
                                    + T * HID * 2, HBM_PEAK)
    total, per, kt = time_steps(torch, step, steps, warmup, 1, table)
    st = float(np.mean(per))
    wl = f"mixed_block_3gdn_1gqa_b{B}" + ("_proj" if proj else "")
    r = dict(workload=wl, tokens_per_step=T, ms_per_step=total / steps * 1e3,
             step_event_ms=st * 1e3, step_event_median_ms=float(np.median(per)) * 1e3, kernels_ms=kt, alg_bytes=bytes_,
             ctx_mean=float(ctx.mean()), ctx_max=int(ctx.max()), verify_tokens=T,
             shape="ctx ~ LogNormal(ln 4096, 1.0) clipped to [256, 65536], 1..4 verify tokens, "
                   f"seed {seed}",
             state="GDN slot pool (shuffled slots), paged KV pool of "
                   f"{int(nblk.sum())} 32-position blocks (interleaved)",
             tok_s=T * steps / total, layer_hbm_gbs=bytes_ / st / 1e9,
             layer_hbm_frac=bytes_ / st / HBM_PEAK,
             roofline=kernel_roofline(kt, table, wl))
    if proj:
        r["proj_flops"] = flops_in + flops_out
        r["proj_weight_bytes"] = 3 * w_gdn + w_att
        if leg:
            r["parity"] = _proj_block_parity(torch, apus_hip, gdn, att, alayer, gpool, slots, rows,
                                             kv, cu, ctx, B, T)
        kpool.destroy()
        gpool.destroy()
        return r
    if leg:
        def slot_states(li):
            conv = torch.empty((B, CD * 3), dtype=torch.int16, device="cuda")
            S = torch.empty((B, HV, DK, DV), dtype=torch.float32, device="cuda")
            for i, sl in enumerate(slots):
                gpool.store_state(li, sl, conv[i], S[i])
            return conv, S
        pre = []
        for li in range(3):
            c0, S0 = slot_states(li)
            torch.cuda.synchronize()
            pre.append((_h16(c0), S0.cpu().numpy()))
        step(0)
        par = {}
        for i, L in enumerate(gdn):
            c1, S1r = slot_states(i)
            S1 = torch.empty_like(S1r)
            apus_hip.gdn_state_pack(S1r, S1)        # the checker unpacks the device layout
            par[f"gdn{i}"] = leg.gdn(torch, L["w"], cu, {n: L[n] for n in ("qkv", "z", "a", "b")},
                                     pre[i][0], pre[i][1], L["y"], c1, S1)
        caches = []
        for s in range(B):
            n = int(ctx[s] + k[s])
            rk = torch.empty((n, NKV, AD), dtype=torch.int16, device="cuda")
            rv = torch.empty_like(rk)
            apus_hip.attn_cache_unpack_paged(kv, rows[s], n, NKV, AD, rk, rv)
            torch.cuda.synchronize()
            caches.append((_h16(rk), _h16(rv)))
        par["attn"] = leg.attn(torch, aw, cu, ctx, {n: att[n] for n in ("qg", "k", "v")}, caches,
                               att["y"])
        par["pass"] = all(v["pass"] for v in par.values())
        par["sample"] = "the whole block step (all 128 sequences, every layer)"
        r["parity"] = par
    kpool.destroy()
    gpool.destroy()
    return r


def _proj_block_parity(torch, apus_hip, gdn, att, alayer, gpool, slots, rows, kv, cu, ctx, B, T):
    """The block with projections against the same block composed of the
    separately checked entry points: from one snapshot of the GDN states
    (and the KV cache, whose appended rows are rewritten with the same
    values), the fused layer calls and the composition (separate MFMA
    GEMMs per weight matrix, the mixer, the output GEMM) must give
    bit-identical outputs and states. The mixers are held to the oracle
    by the c4 line and the GEMMs by the test suite; the layer calls are
    held to both, stage by stage, in tests/test_gpu_layer.py."""
    snaps = []
    for li in range(3):
        conv = torch.empty((B, CD * 3), dtype=torch.int16, device="cuda")
        S = torch.empty((B, HV, DK, DV), dtype=torch.float32, device="cuda")
        for i, sl in enumerate(slots):
            gpool.store_state(li, sl, conv[i], S[i])
        snaps.append((conv, S))

    def restore():
        for li, (conv, S) in enumerate(snaps):
            for i, sl in enumerate(slots):
                gpool.load_state(li, sl, conv[i], S[i])

    def run_fused():
        for L in gdn:
            apus_hip.gdn_layer_decode_slots(L["layer"], L["proj"], slots, slots, cu, L["ln1"],
                                            L["conv"], L["S"], L["ao"])
        apus_hip.attn_layer_decode_paged(alayer, att["proj"], rows, cu, ctx, att["ln1"], kv,
                                         att["ao"])
        return [L["ao"].clone() for L in gdn] + [att["ao"].clone()]

    def run_composed():
        outs = []
        for L in gdn:
            P = L["pw"]
            for wn, dst in (("w_qkv", "qkv"), ("w_z", "z"), ("w_b", "b"), ("w_a", "a")):
                apus_hip.bf16_gemm_dev(P[wn], L["ln1"], L[dst], exact=False)
            apus_hip.gdn_decode_slots(L["layer"], slots, slots, cu, L["qkv"], L["z"], L["a"],
                                      L["b"], L["conv"], L["S"], L["y"])
            o = torch.empty_like(L["ao"])
            apus_hip.bf16_gemm_dev(P["w_out"], L["y"], o, exact=False)
            outs.append(o)
        P = att["pw"]
        for wn, dst in (("wq", "qg"), ("wk", "k"), ("wv", "v")):
            apus_hip.bf16_gemm_dev(P[wn], att["ln1"], att[dst].view(T, -1), exact=False)
        apus_hip.attn_decode_paged(alayer, rows, cu, ctx, att["qg"], att["k"], att["v"], kv,
                                   att["y"])
        o = torch.empty_like(att["ao"])
        apus_hip.bf16_gemm_dev(P["wo"], att["y"], o, exact=False)
        outs.append(o)
        return outs

    def states():
        out = []
        for li in range(3):
            conv = torch.empty((B, CD * 3), dtype=torch.int16, device="cuda")
            S = torch.empty((B, HV, DK, DV), dtype=torch.float32, device="cuda")
            for i, sl in enumerate(slots):
                gpool.store_state(li, sl, conv[i], S[i])
            out.append((conv, S))
        return out

    restore()
    fused = run_fused()
    fused_states = states()
    restore()
    comp = run_composed()
    comp_states = states()
    torch.cuda.synchronize()
    same = [bool(torch.equal(a, b)) for a, b in zip(fused, comp)]
    same_state = all(bool(torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]))
                     for a, b in zip(fused_states, comp_states))
    return {"pass": all(same) and same_state, "layers_bitwise": same,
            "states_bitwise": same_state,
            "check": "fused layer calls == separate GEMM + mixer + GEMM launches, bit for bit "
                     "(every stage held to the oracle in tests/test_gpu_layer.py)"}


PROJ_O, PROJ_K = CD + VD + 2 * HV, 2048   # GDN in_proj: qkv | z | a | b (12352 x 2048)


def bench_proj(torch, M, exact, steps, warmup, seed):
    """The GDN layer's input projection (the step on the path's input
    side): y [M, 12352] = x [M, 2048] . w^T, bf16. exact: the
    reference-order kernel (bitwise, decode-sized M); else the MFMA GEMM.
    Weight sets rotate so the 50 MB weight is read from HBM."""
    import apus_hip
    O, K = PROJ_O, PROJ_K
    nsets = 6
    g = torch.Generator(device="cuda").manual_seed(seed)
    sets = []
    for _ in range(nsets):
        w = (torch.randn((O, K), generator=g, device="cuda") * K ** -0.5).to(torch.bfloat16)
        x = torch.randn((M, K), generator=g, device="cuda").to(torch.bfloat16)
        y = torch.empty((M, O), dtype=torch.bfloat16, device="cuda")
        sets.append((w.view(torch.int16), x.view(torch.int16), y.view(torch.int16)))

    def step(i):
        w, x, y = sets[i]
        apus_hip.bf16_gemm_dev(w, x, y, exact=exact)

    kname = "k_gemm_seq" if exact else "k_gemm_tile"
    bytes_ = O * K * 2 + M * K * 2 + M * O * 2
    flops = 2 * M * O * K
    table = {kname: ("hbm", bytes_, HBM_PEAK) if M <= 256 else ("mfma", flops, BF16_PEAK)}
    total, per, kt = time_steps(torch, step, steps, warmup, nsets, table)
    wl = f"gdn_in_proj_m{M}"
    return dict(workload=wl, tokens_per_step=M, ms_per_step=total / steps * 1e3,
                step_event_ms=float(np.mean(per)) * 1e3, step_event_median_ms=float(np.median(per)) * 1e3, kernels_ms=kt, alg_bytes=bytes_,
                alg_flops=flops, exact=exact, tok_s=M * steps / total,
                roofline=kernel_roofline(kt, table, wl))


def bench_copy(torch, steps, warmup):
    """Calibration workload for HBM counters: a plain 1 GiB device copy
    (reads 1 GiB, writes 1 GiB); rocprofv3 FETCH_SIZE / WRITE_SIZE of its
    kernel against 1,048,576 KiB give the counter scale."""
    n = 1 << 30
    a = [torch.empty(n, dtype=torch.uint8, device="cuda") for _ in range(2)]
    b = [torch.empty(n, dtype=torch.uint8, device="cuda") for _ in range(2)]
    for x in a:
        x.fill_(1)

    def step(i):
        b[i].copy_(a[i])

    total, per, _ = time_steps(torch, step, steps, warmup, 2)
    st = float(np.mean(per))
    return dict(workload="copy_1GiB", ms_per_step=total / steps * 1e3, step_event_ms=st * 1e3, step_event_median_ms=float(np.median(per)) * 1e3,
                alg_bytes=2 * n, hbm_gbs=2 * n / st / 1e9, tok_s=0.0)


# ---------------------------------------------------------------- CPU side
def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def _cgroup_cpus():
    """CPUs granted by the cgroup quota (cpu.max), or None when unlimited."""
    try:
        q, p = open("/sys/fs/cgroup/cpu.max").read().split()
        return None if q == "max" else max(1, int(int(q) / int(p)))
    except (OSError, ValueError):
        return None


def _avail_cores():
    """Cores this process may use: the affinity mask, capped by a cgroup
    quota when one is set."""
    n = len(os.sched_getaffinity(0))
    q = _cgroup_cpus()
    return min(n, q) if q else n


REF_POOL_MAX = 32          # the reference pool's lane cap (c/pool.h:52)
CPU_CONFIGS = ("c0", "c0b", "c1", "c2", "c3", "c4")


def _code_pool(rng, n):
    """Finite bf16 codes with |x| in [2^-31, 2) and random signs."""
    return (rng.integers(0x3000, 0x4000, n, dtype=np.uint16)
            | (rng.integers(0, 2, n, dtype=np.uint16) << 15)).astype(np.uint16)


def cpu_worker(threads):
    """Child process (APUS_THREADS / OMP_NUM_THREADS = threads): time each
    configuration's bounded sample on the oracle port (the C restatement
    of the reference's anchors) and print one JSON
    line per configuration: seconds measured, and the config's tokens per
    second derived from them (rule in "rule")."""
    import oracle
    import synth
    # the repo's C restatement of the anchors (pinned bitwise to the
    # reference's own c/gdn.h / c/attn.h in the CPU tests); reference code
    # itself never travels to the GPU box
    lib = oracle.Oracle()
    kind = "port"
    kw = dict(nthreads=threads)
    rng = np.random.default_rng(1)
    w = synth.gdn_weights(rng)
    aw = synth.attn_weights(rng)

    def gdn(B, T, zero):
        tok = synth.gdn_tokens(rng, B * T)
        conv, S = synth.gdn_state(rng, B, zero=zero)
        cu = np.arange(B + 1, dtype=np.int32) * T
        return lambda: lib.gdn_mixer(GDN, w, cu, tok["qkv"], tok["z"], tok["a"], tok["b"], conv, S,
                                     **kw)

    def attn(ctx, k, pool):
        """B sequences with ctx[s] cached tokens (cache rows sliced from a
        shared code pool) verifying k[s] new ones, run one sequence after
        another as the reference engine does."""
        calls = []
        for c, n in zip(ctx, k):
            rows = int(c) + int(n)
            o = int(rng.integers(0, pool.size - 2 * rows * NKV * AD))
            kc = pool[o:o + rows * NKV * AD]
            vc = pool[o + rows * NKV * AD:o + 2 * rows * NKV * AD]
            tok = synth.attn_tokens(rng, int(n))
            cu1 = np.array([0, int(n)], np.int32)
            p0 = np.array([int(c)], np.int32)
            calls.append((cu1, p0, tok, kc, vc, rows))

        def run():
            for cu1, p0, tok, kc, vc, rows in calls:
                lib.attn_mixer(ATTN, aw, cu1, p0, tok["qg"], tok["k"], tok["v"], kc, vc,
                               rows * NKV * AD, **kw)
        return run

    def timed(fn, reps=1, warm=False):
        if warm:
            fn()                               # pool spawn, page faults
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        return (time.perf_counter() - t0) / reps

    pool = _code_pool(rng, 48 << 20)
    out = {}
    t = timed(gdn(1, 1, False), reps=20, warm=True)
    out["c0"] = dict(seconds=t, tok_s=1 / t, rule="one decode token, batch 1, 20 repetitions")
    t = timed(gdn(64, 1, False))
    out["c0b"] = dict(seconds=t, tok_s=64 / t, rule="64 sequences, one token each (full config)")
    t = timed(gdn(1, 256, True))
    out["c1"] = dict(seconds=t, tok_s=256 / t,
                     rule="256 prompt tokens from zero state; the reference's prefill runs its "
                          "per-token loop (c/layer.h:454-489), so the per-token cost and the rate "
                          "do not depend on T")
    t = timed(attn([32767] * 2, [1] * 2, pool))
    out["c2"] = dict(seconds=t, tok_s=2 / t,
                     rule="2 of the 64 sequences (each 32767 cached + 1 new); every sequence is "
                          "the same work, run one after another")
    t = timed(attn([0], [512], pool))
    scale = (8192 * 8193) / (512 * 513)
    out["c3"] = dict(seconds=t, tok_s=8192 / (t * scale),
                     rule="T=512 from position 0, time scaled to T=8192 by the causal pair count "
                          f"(x{scale:.1f}: attention dominates; norm/rope/append are linear)")
    ctx, k = synth.mixed_block_shape(128, 15)
    cu = np.concatenate([[0], np.cumsum(k)]).astype(np.int32)
    g3 = []
    for _ in range(3):
        tok = synth.gdn_tokens(rng, int(k.sum()))
        conv, S = synth.gdn_state(rng, len(k))
        g3.append((tok, conv, S))

    def gdn3():
        for tok, conv, S in g3:
            lib.gdn_mixer(GDN, w, cu, tok["qkv"], tok["z"], tok["a"], tok["b"], conv, S, **kw)
    t_g = timed(gdn3)
    # attention on every 8th sequence in context order, scaled by the
    # (new tokens x keys) work of the whole batch
    order = np.argsort(ctx)[4::8]
    work = lambda idx: float(np.sum(k[idx].astype(np.float64) * (ctx[idx] + k[idx])))
    t_a = timed(attn(ctx[order], k[order], pool)) * work(np.arange(len(k))) / work(order)
    t = t_g + t_a
    out["c4"] = dict(seconds=t, tok_s=float(k.sum()) / t,
                     rule="3 GDN mixers over all 128 sequences (325 verify tokens) timed whole; the "
                          "GQA mixer timed on 16 of the sequences (every 8th by context) and scaled "
                          "by the batch's sum of new tokens x keys")
    print(json.dumps(dict(kind=kind, threads=threads, configs=out)))


def cpu_baseline(head):
    """Time the CPU samples at min(32, cores) and at all usable cores (one
    child process each: the reference pool fixes its lanes at first use)."""
    n = _avail_cores()
    runs = []
    for th in sorted({min(REF_POOL_MAX, n), n}):
        env = dict(os.environ, APUS_THREADS=str(th), OMP_NUM_THREADS=str(th))
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-worker",
                            "--cpu-threads", str(th)], env=env, capture_output=True, text=True,
                           timeout=900)
        if r.returncode != 0:
            log("cpu baseline failed:", r.stderr[-2000:])
            continue
        runs.append(json.loads(r.stdout.strip().splitlines()[-1]))
        log("cpu", runs[-1])
    if not runs:
        return None
    first = runs[0]
    c = first["configs"][head]
    return dict(value=c["tok_s"], unit="tok/s", cores=first["threads"], kind=first["kind"],
                sample=(f"config {head}: {c['rule']}; "
                        "the repo oracle port (oracle/apus_oracle.c, bitwise-pinned to c/gdn.h + c/attn.h)"
                        f" with {first['threads']} threads on {cpu_model()}"),
                nproc=os.cpu_count(), usable_cores=n, cgroup_cpus=_cgroup_cpus(),
                cpu_model=cpu_model(),
                runs={f"{x['kind']}@{x['threads']}": {k: dict(tok_s=v["tok_s"], seconds=v["seconds"])
                                                      for k, v in x["configs"].items()} for x in runs},
                rules={k: v["rule"] for k, v in first["configs"].items()})


def _rounded(x):
    if isinstance(x, dict):
        return {k: _rounded(v) for k, v in x.items()}
    if isinstance(x, list):
        return [_rounded(v) for v in x]
    if isinstance(x, float):
        return float(f"{x:.6g}")
    return x


TOLERANCE_READING = (
    "north star 'max relative error <= 2e-3 on bf16 outputs' read as the normwise relative error "
    "over each output tensor (parity.rel); per element the tests (tests/) hold GDN decode to 1 bf16 "
    "ulp, GDN prefill to 4 ulps (row-RMS floor), GQA to 2e-3 of (|r| + sum |terms|) plus rounding "
    "flips within the fp32 summation bound or 2 ulps; '<= 1e-4 on the fp32 state' as "
    "max|S - S_ref| / max|S_ref| (parity.state_rel); caches and conv states bit-exact")


# ---------------------------------------------------------------- main
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--only", default="c0,c0b,c1,c2,c3,c4,c4p,p1,p64,p4096")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--cpu-worker", action="store_true")
    args = ap.parse_args()
    if args.cpu_worker:
        cpu_worker(args.cpu_threads)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the mixers shard by sequence or by head with no exchange inside the path). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import apus_hip
    apus_hip.init(0)
    apus_hip.set_stream(torch.cuda.current_stream().cuda_stream)
    want = set(args.only.split(","))
    leg = None if args.no_cpu else CpuLeg()
    res = {}
    runs = (("c0", lambda: bench_gdn_decode(torch, 1, max(args.steps, 50), args.warmup, 10, leg)),
            ("c0b", lambda: bench_gdn_decode(torch, 64, args.steps, args.warmup, 11, leg)),
            ("c1", lambda: bench_gdn_prefill(torch, 4096, args.steps, args.warmup, 12, leg)),
            ("c2", lambda: bench_attn_decode(torch, 64, 32768, args.steps, args.warmup, 13, leg)),
            ("c3", lambda: bench_attn_prefill(torch, 8192, args.steps, args.warmup, 14, leg)),
            ("c4", lambda: bench_mixed_block(torch, 128, args.steps, args.warmup, 15, leg)),
            ("c4p", lambda: bench_mixed_block(torch, 128, args.steps, args.warmup, 15, leg,
                                              proj=True)),
            ("p1", lambda: bench_proj(torch, 1, True, args.steps, args.warmup, 16)),
            ("p64", lambda: bench_proj(torch, 64, False, args.steps, args.warmup, 16)),
            ("p4096", lambda: bench_proj(torch, 4096, False, args.steps, args.warmup, 16)),
            ("copy", lambda: bench_copy(torch, args.steps, args.warmup)))
    for name, fn in runs:
        if name in want:
            res[name] = fn()
            log(name, json.dumps(_rounded(res[name])))
            torch.cuda.empty_cache()

    hk = "c4" if "c4" in res else next((k for k, v in res.items() if "roofline" in v), None)
    if hk is None:                       # calibration-only run
        print(json.dumps(dict(metric="copy calibration", configs=_rounded(res))))
        return
    head = res[hk]
    cpu = None if args.no_cpu else cpu_baseline(hk if hk in CPU_CONFIGS else "c4")
    line = dict(metric="attn-layer tok/s @1 GPU; decode HBM GB/s % peak; prefill MFMA TFLOP/s % peak",
                value=head["tok_s"], unit="tok/s", n_gpus=1, steps=args.steps, warmup=args.warmup,
                ms_per_step=head["ms_per_step"], higher_is_better=True, scaling="weak",
                vs_baseline=None, dtype="f32",
                data="synthetic (bf16 storage, fp32 arithmetic; bf16 MFMA with fp32 accumulation "
                     "in the attention products)",
                config=dict(workload=head["workload"], global_batch=head["tokens_per_step"],
                            seq_len=head.get("ctx_max", head["tokens_per_step"]),
                            parallelism="none (1 GPU)"),
                roofline=head["roofline"], cpu_baseline=cpu, parity=head.get("parity"),
                tolerance_reading=TOLERANCE_READING,
                configs=res)
    print(json.dumps(_rounded(line)))


if __name__ == "__main__":
    main()
