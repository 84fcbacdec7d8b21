"""Benchmark of the apus-qwen attention hot path on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--only c0,c0b,c1,...]
                [--no-cpu]

A "step" is one pass of a mixer (the hot path between a layer's input
projections and its output projection) over one batch of synthetic inputs
already resident in HBM. The headline line is BASELINE config 1 (Gated
DeltaNet prefill, batch 1, T=4096, zero initial state), reported as tokens
per second; the other configurations are measured in the same run and
reported under "configs" with their own roofline fractions:
  c0   config 0   GDN decode, batch 1
  c0b  config 0'  GDN decode, batch 64 (HBM-bound decode)
  c1   config 1   GDN prefill T=4096 (headline)
  c2   config 2   gated-GQA decode, 64 sequences x 32K-token bf16 KV cache
  c3   config 3   gated-GQA causal prefill, T=8192 (cache fill + attention)
  c4   config 4   hybrid decode block, 3 GDN + 1 GQA layers, 128 sequences
                  verifying 1..4 tokens each at log-normal cached contexts
  p1, p64, p4096  the GDN input projection (2048 -> 12352) beside the path:
                  1 token (reference-order kernel, bitwise), 64 tokens
                  (MFMA GEMM), 4096 tokens (rocBLAS bf16 GEMM)
Input buffer sets rotate so the 256 MB Infinity Cache cannot serve
repeated reads. The CPU baseline is the reference's own scalar anchors
(oracle/_ref, built from the reference sources) when present, else the
repo's C restatement (oracle/), timed on the host cores on a bounded sample.
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
for p in (PKG, os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK = 8.0e12            # B/s, MI355X HBM3E
BF16_PEAK = 2.5e15           # flop/s dense bf16 MFMA
FP32_PEAK = 157.3e12         # flop/s dense fp32 MFMA
CPU_THREADS = 16             # the GPU box's CPU share for one GPU

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
    i % nsets. The wall-clock pass runs without kernel timing; a second
    pass of the same steps records HIP events around each launch of the
    named kernels on the library's stream (apus_hip_timing_*)."""
    import apus_hip
    for i in range(warmup):
        fn(i % nsets)
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        ev[i][0].record()
        fn(i % nsets)
        ev[i][1].record()
    torch.cuda.synchronize()
    total = time.perf_counter() - t0
    per = [a.elapsed_time(b) * 1e-3 for a, b in ev]
    kt = {}
    if kernels:
        apus_hip.timing_enable(True)
        for i in range(steps):
            fn(i % nsets)
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
    """Roofline of the dominant kernel: table maps kernel name to
    (bound, algorithmic units per launch, peak per second); achieved =
    units / that kernel's average launch time."""
    name = max((k for k in table if k in kt), key=lambda k: kt[k])
    bound, units, peak = table[name]
    sec = kt[name] * 1e-3
    traffic = measured_traffic(workload, name)
    if bound == "mfma":
        return dict(kernel=name, bound="mfma", achieved=units / sec / 1e12, peak=peak / 1e12,
                    unit="TFLOP/s", frac=units / sec / peak, traffic=traffic, launch_ms=kt[name],
                    per_launch=units)
    return dict(kernel=name, bound="hbm", achieved=units / sec / 1e9, peak=peak / 1e9,
                unit="GB/s", frac=units / sec / peak, traffic=traffic, launch_ms=kt[name],
                per_launch=units)


# ---------------------------------------------------------------- workloads
def bench_gdn_decode(torch, B, steps, warmup, seed):
    """Config 0 / 0': one decode token per sequence, prior state."""
    import apus_hip
    nsets = 4 if B > 1 else 8
    d = Dev(torch, B, 1, nsets, seed, zero_state=False)

    def step(i):
        s = d.sets[i]
        apus_hip.gdn_decode(d.layer, d.cu, s["qkv"], s["z"], s["a"], s["b"], s["conv"], s["S"], s["y"])

    bytes_ = B * gdn_seq_bytes(1) + GDN_WEIGHT_BYTES
    table = {"k_gdn_decode": ("hbm", bytes_, HBM_PEAK)}
    total, per, kt = time_steps(torch, step, steps, warmup, nsets, table)
    st = float(np.mean(per))
    wl = f"gdn_decode_b{B}"
    return dict(workload=wl, tokens_per_step=B, ms_per_step=total / steps * 1e3,
                step_event_ms=st * 1e3, kernels_ms=kt, alg_bytes=bytes_,
                tok_s=B * steps / total, roofline=kernel_roofline(kt, table, wl))


def bench_gdn_prefill(torch, T, steps, warmup, seed):
    """Config 1: one sequence of T tokens from zero state."""
    import apus_hip
    nsets = 2
    d = Dev(torch, 1, T, nsets, seed, zero_state=True)

    def step(i):
        s = d.sets[i]
        s["conv"].zero_()
        s["S"].zero_()
        apus_hip.gdn_prefill(d.layer, d.cu, s["qkv"], s["z"], s["a"], s["b"], s["conv"], s["S"], s["y"])

    bytes_ = gdn_seq_bytes(T) + GDN_WEIGHT_BYTES
    flops = gdn_prefill_flops(T)
    nu = (T // 64) * HV                       # (chunk, v-head) units
    # the scan multiplies fp32 operands on the bf16 MFMA in split precision
    # (hi*hi + hi*lo + lo*hi: three bf16 MFMAs per fp32 product), so its roof
    # for the fp32 algorithm is a third of the bf16 peak
    table = {"k_gdn_chunk_scan": ("mfma", nu * SCAN_FLOPS_PER_UNIT, BF16_PEAK / 3),
             "k_gdn_chunk_wy": ("mfma", nu * WY_FLOPS_PER_UNIT, FP32_PEAK),
             "k_gdn_prep": ("hbm", gdn_prep_bytes(T), HBM_PEAK),
             "k_gdn_post": ("hbm", gdn_post_bytes(T), HBM_PEAK)}
    total, per, kt = time_steps(torch, step, steps, warmup, nsets, table)
    st = float(np.mean(per))
    wl = f"gdn_prefill_t{T}"
    return dict(workload=wl, tokens_per_step=T, ms_per_step=total / steps * 1e3,
                step_event_ms=st * 1e3, kernels_ms=kt, alg_bytes=bytes_, alg_flops=flops,
                tok_s=T * steps / total, layer_hbm_frac=bytes_ / st / HBM_PEAK,
                layer_tflops=flops / st / 1e12, roofline=kernel_roofline(kt, table, wl))


# Algorithmic flops per (chunk of 64, v-head) of the two chunk kernels:
# the scan does W S0, Q S0, K^T D (64x128x128 each) and A D (64x64x128);
# the WY build does K K^T, Q K^T (64x64x128) and the two 64x64x128
# triangular applications giving U and W, plus the triangular solve.
SCAN_FLOPS_PER_UNIT = 3 * 2 * 64 * 128 * 128 + 2 * 64 * 64 * 128
WY_FLOPS_PER_UNIT = 4 * 2 * 64 * 64 * 128 + (2 * 64 ** 3) // 3


def gdn_prep_bytes(T):
    """k_gdn_prep interface bytes: qkv, a, b in; fp32 l2-normed q and k,
    conv+SiLU v (bf16), (exp g, beta) and g out; old conv state in."""
    return T * (CD * 2 + HV * 2 * 2 + 2 * HK * DK * 4 + VD * 2 + HV * 8 + HV * 4) + CD * 3 * 2


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


def attn_decode_bytes(ctx, tq=1):
    """Algorithmic HBM bytes of one sequence's decode step: the K and V
    cache rows read (ctx keys x nkv x d x 2 B each), the new q|gate, k, v
    read, the appended k, v written, and the gated output written."""
    kv = ctx * NKV * AD * 2 * 2
    per_tok = NH * 2 * AD * 2 + NKV * AD * 2 * 2 + NKV * AD * 2 * 2 + NH * AD * 2
    return kv + tq * per_tok


def bench_attn_decode(torch, B, ctx, steps, warmup, seed):
    """Config 2: B sequences, each with ctx-1 cached tokens plus one new
    token (so the new token attends ctx keys)."""
    import apus_hip
    dev = torch.device("cuda")
    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def bf(shape, std=1.0):
        return (torch.randn(shape, generator=g, device=dev) * std).to(torch.bfloat16).view(torch.int16)

    w = dict(qn_w=bf((AD,), 0.1), kn_w=bf((AD,), 0.1))
    layer = apus_hip.attn_layer(ATTN, w)
    max_seq = ctx
    kc = bf((B, NKV, max_seq, AD))
    vc = bf((B, NKV, max_seq // 32, AD, 32))
    nsets = 2
    sets = [dict(qg=bf((B, NH, 2 * AD)), k=bf((B, NKV, AD)), v=bf((B, NKV, AD)),
                 y=torch.empty((B, NH * AD), dtype=torch.int16, device=dev)) for _ in range(nsets)]
    cu = np.arange(B + 1, dtype=np.int32)
    pos0 = np.full(B, ctx - 1, np.int32)

    def step(i):
        s = sets[i]
        apus_hip.attn_decode(layer, cu, pos0, s["qg"], s["k"], s["v"], kc, vc, max_seq, s["y"])

    bytes_ = B * attn_decode_bytes(ctx) + 2 * AD * 2
    flops = B * NH * 4 * AD * ctx
    kbytes = B * ctx * NKV * AD * 2           # one of the K / V caches
    table = {"k_attn_scores": ("hbm", kbytes, HBM_PEAK), "k_attn_pv": ("hbm", kbytes, HBM_PEAK),
             "k_attn_prep": ("hbm", B * (NH * AD * 2 * 2 + NKV * AD * 2 * 2), HBM_PEAK),
             "k_attn_vappend": ("hbm", B * NKV * AD * 2 * 2, HBM_PEAK),
             "k_attn_combine": ("hbm", B * NH * AD * 2 * 2, HBM_PEAK)}
    total, per, kt = time_steps(torch, step, steps, warmup, nsets, table)
    st = float(np.mean(per))
    wl = f"attn_decode_b{B}_ctx{ctx}"
    return dict(workload=wl, tokens_per_step=B, ms_per_step=total / steps * 1e3,
                step_event_ms=st * 1e3, kernels_ms=kt, alg_bytes=bytes_, alg_flops=flops,
                tok_s=B * steps / total, layer_hbm_gbs=bytes_ / st / 1e9,
                layer_hbm_frac=bytes_ / st / HBM_PEAK, roofline=kernel_roofline(kt, table, wl))


def attn_prefill_flops(T):
    """Causal GQA prefill, algorithmic: q.k and P.V over the keys each row
    sees (16 heads x 256 dims x 2 flop x 2 matmuls x T(T+1)/2 rows-keys)."""
    return NH * 4 * AD * (T * (T + 1) // 2)


def bench_attn_prefill(torch, T, steps, warmup, seed):
    """Config 3: one sequence, T new tokens from position 0: norm, RoPE,
    cache fill and causal attention with the output gate."""
    import apus_hip
    dev = torch.device("cuda")
    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def bf(shape, std=1.0):
        return (torch.randn(shape, generator=g, device=dev) * std).to(torch.bfloat16).view(torch.int16)

    w = dict(qn_w=bf((AD,), 0.1), kn_w=bf((AD,), 0.1))
    layer = apus_hip.attn_layer(ATTN, w)
    nsets = 2
    sets = [dict(qg=bf((T, NH, 2 * AD)), k=bf((T, NKV, AD)), v=bf((T, NKV, AD)),
                 kc=torch.empty((1, NKV, T, AD), dtype=torch.int16, device=dev),
                 vc=torch.empty((1, NKV, T // 32, AD, 32), dtype=torch.int16, device=dev),
                 y=torch.empty((T, NH * AD), dtype=torch.int16, device=dev)) for _ in range(nsets)]
    cu = np.array([0, T], np.int32)
    pos0 = np.zeros(1, np.int32)

    def step(i):
        s = sets[i]
        apus_hip.attn_prefill(layer, cu, pos0, s["qg"], s["k"], s["v"], s["kc"], s["vc"], T, s["y"])

    flops = attn_prefill_flops(T)
    bytes_ = T * (NH * 2 * AD * 2 + 2 * NKV * AD * 2 + 2 * NKV * AD * 2 + NH * AD * 2)
    table = {"k_attn_fa": ("mfma", flops, BF16_PEAK),
             # q and k rows read and written (normed, roped), v rows appended
             "k_attn_prep": ("hbm", T * (NH * AD * 2 * 2 + NKV * AD * 2 * 2), HBM_PEAK),
             "k_attn_vappend": ("hbm", T * NKV * AD * 2 * 2, HBM_PEAK)}
    total, per, kt = time_steps(torch, step, steps, warmup, nsets, table)
    st = float(np.mean(per))
    wl = f"attn_prefill_t{T}"
    return dict(workload=wl, tokens_per_step=T, ms_per_step=total / steps * 1e3,
                step_event_ms=st * 1e3, kernels_ms=kt, alg_bytes=bytes_, alg_flops=flops,
                tok_s=T * steps / total, layer_tflops=flops / st / 1e12,
                layer_mfma_frac=flops / st / BF16_PEAK, roofline=kernel_roofline(kt, table, wl))


def bench_mixed_block(torch, B, steps, warmup, seed):
    """Config 4: one hybrid decode block in the model's 3:1 ratio -- three
    Gated DeltaNet layers (each with its own weights, conv state and
    recurrent state per sequence) and one gated-GQA layer (a bf16 KV cache
    per sequence) -- over B sequences that each verify 1..4 tokens at a
    log-normal cached context. value = verified tokens per second through
    the block."""
    import apus_hip
    dev = torch.device("cuda")
    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def bf(shape, std=1.0, mean=0.0):
        x = torch.randn(shape, generator=g, device=dev, dtype=torch.float32) * std + mean
        return x.to(torch.bfloat16).view(torch.int16)

    import synth
    ctx, k = synth.mixed_block_shape(B, seed)
    cu = np.concatenate([[0], np.cumsum(k)]).astype(np.int32)
    T = int(cu[-1])
    gdn = []
    for _ in range(3):
        w = dict(conv_w=bf((CD, 4), 0.1), A_log=torch.rand(HV, generator=g, device=dev) * 2.7,
                 dt_bias=torch.ones(HV, device=dev), onorm_w=bf((DV,), 0.1, 1.0))
        gdn.append(dict(layer=apus_hip.gdn_layer(GDN, w), w=w, qkv=bf((T, CD)), z=bf((T, VD)),
                        a=bf((T, HV)), b=bf((T, HV)), conv=bf((B, CD * 3)),
                        S=torch.randn((B, HV, DK, DV), generator=g, device=dev) * 0.02,
                        y=torch.empty((T, VD), dtype=torch.int16, device=dev)))
    aw = dict(qn_w=bf((AD,), 0.1), kn_w=bf((AD,), 0.1))
    alayer = apus_hip.attn_layer(ATTN, aw)
    max_seq = int(-(-int((ctx + k).max()) // 32) * 32)
    # caches filled with finite random bf16 codes (|x| < 1) without an fp32
    # temporary of the caches' size
    kc = torch.randint(-16000, 16000, (B, NKV, max_seq, AD), dtype=torch.int16, device=dev, generator=g)
    vc = torch.randint(-16000, 16000, (B, NKV, max_seq // 32, AD, 32), dtype=torch.int16, device=dev,
                       generator=g)
    att = dict(qg=bf((T, NH, 2 * AD)), k=bf((T, NKV, AD)), v=bf((T, NKV, AD)),
               y=torch.empty((T, NH * AD), dtype=torch.int16, device=dev))

    def step(i):
        for L in gdn:
            apus_hip.gdn_decode(L["layer"], cu, L["qkv"], L["z"], L["a"], L["b"], L["conv"],
                                L["S"], L["y"])
        apus_hip.attn_decode(alayer, cu, ctx, att["qg"], att["k"], att["v"], kc, vc, max_seq,
                             att["y"])

    gdn_bytes = sum(gdn_seq_bytes(int(x)) for x in k) + GDN_WEIGHT_BYTES
    attn_bytes = sum(attn_decode_bytes(int(c) + int(x), int(x)) for c, x in zip(ctx, k)) + 2 * AD * 2
    bytes_ = 3 * gdn_bytes + attn_bytes
    kv1 = int(sum((int(c) + int(x)) * NKV * AD * 2 for c, x in zip(ctx, k)))   # one of K / V
    table = {"k_gdn_decode": ("hbm", gdn_bytes, HBM_PEAK),
             "k_attn_scores": ("hbm", kv1, HBM_PEAK), "k_attn_pv": ("hbm", kv1, HBM_PEAK),
             "k_attn_prep": ("hbm", T * (NH * AD * 2 * 2 + NKV * AD * 2 * 2), HBM_PEAK),
             "k_attn_vappend": ("hbm", T * NKV * AD * 2 * 2, HBM_PEAK),
             "k_attn_combine": ("hbm", T * NH * AD * 2 * 2, HBM_PEAK)}
    total, per, kt = time_steps(torch, step, steps, warmup, 1, table)
    st = float(np.mean(per))
    wl = f"mixed_block_3gdn_1gqa_b{B}"
    return dict(workload=wl, tokens_per_step=T, ms_per_step=total / steps * 1e3,
                step_event_ms=st * 1e3, kernels_ms=kt, alg_bytes=bytes_,
                ctx_mean=float(ctx.mean()), ctx_max=int(ctx.max()), verify_tokens=T,
                tok_s=T * steps / total, layer_hbm_gbs=bytes_ / st / 1e9,
                layer_hbm_frac=bytes_ / st / HBM_PEAK,
                roofline=kernel_roofline(kt, table, wl))


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

    kname = "k_gemm_seq" if exact else ("k_gemm_mfma" if M <= 256 else "rocblas_gemm_bf16")
    bytes_ = O * K * 2 + M * K * 2 + M * O * 2
    flops = 2 * M * O * K
    table = {kname: ("hbm", bytes_, HBM_PEAK) if M <= 256 else ("mfma", flops, BF16_PEAK)}
    total, per, kt = time_steps(torch, step, steps, warmup, nsets, table)
    wl = f"gdn_in_proj_m{M}"
    return dict(workload=wl, tokens_per_step=M, ms_per_step=total / steps * 1e3,
                step_event_ms=float(np.mean(per)) * 1e3, kernels_ms=kt, alg_bytes=bytes_,
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
    return dict(workload="copy_1GiB", ms_per_step=total / steps * 1e3, step_event_ms=st * 1e3,
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


def cpu_baseline_worker(args):
    """Runs in a child process with APUS_THREADS / OMP_NUM_THREADS set:
    the config 1 mixer over a T-token sample, continuing state."""
    import oracle
    import synth
    rng = np.random.default_rng(1)
    T = args.cpu_tokens
    w = synth.gdn_weights(rng)
    tok = synth.gdn_tokens(rng, T)
    conv, S = synth.gdn_state(rng, 1, zero=True)
    cu = np.array([0, T], np.int32)
    if oracle.Reference.available():
        lib, kind = oracle.Reference(), "reference"
        run = lambda: lib.gdn_mixer(GDN, w, cu, tok["qkv"], tok["z"], tok["a"], tok["b"], conv, S)
    else:
        lib, kind = oracle.Oracle(), "port"
        run = lambda: lib.gdn_mixer(GDN, w, cu, tok["qkv"], tok["z"], tok["a"], tok["b"], conv, S,
                                    nthreads=args.cpu_threads)
    run()   # warm (thread pool spawn, page faults)
    t0 = time.perf_counter()
    run()
    dt = time.perf_counter() - t0
    print(json.dumps(dict(kind=kind, seconds=dt, tokens=T)))


def cpu_baseline(threads, tokens):
    env = dict(os.environ, APUS_THREADS=str(threads), OMP_NUM_THREADS=str(threads))
    r = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-worker",
                        "--cpu-tokens", str(tokens), "--cpu-threads", str(threads)],
                       env=env, capture_output=True, text=True, timeout=600)
    if r.returncode != 0:
        log("cpu baseline failed:", r.stderr[-2000:])
        return None
    res = json.loads(r.stdout.strip().splitlines()[-1])
    return dict(value=tokens / res["seconds"], unit="tok/s", cores=threads, kind=res["kind"],
                sample=(f"config 1 GDN mixer (conv, beta, decay, l2norm, step_mt, rnd, onorm per "
                        f"token) over {tokens} tokens from zero state, batch 1, "
                        f"{'reference c/gdn.h anchors' if res['kind'] == 'reference' else 'oracle port'}"
                        f" with {threads} pool threads on {cpu_model()} (nproc {os.cpu_count()})"))


def _rounded(x):
    if isinstance(x, dict):
        return {k: _rounded(v) for k, v in x.items()}
    if isinstance(x, float):
        return float(f"{x:.6g}")
    return x


# ---------------------------------------------------------------- main
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--only", default="c0,c0b,c1,c2,c3,c4,p1,p64,p4096")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-tokens", type=int, default=8192)
    ap.add_argument("--cpu-threads", type=int, default=CPU_THREADS)
    ap.add_argument("--cpu-worker", action="store_true")
    args = ap.parse_args()
    if args.cpu_worker:
        cpu_baseline_worker(args)
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
    res = {}
    if "c0" in want:
        res["c0"] = bench_gdn_decode(torch, 1, max(args.steps, 50), args.warmup, 10)
        log("c0", res["c0"])
    if "c0b" in want:
        res["c0b"] = bench_gdn_decode(torch, 64, args.steps, args.warmup, 11)
        log("c0b", res["c0b"])
    if "c1" in want:
        res["c1"] = bench_gdn_prefill(torch, 4096, args.steps, args.warmup, 12)
        log("c1", res["c1"])

    if "c2" in want:
        res["c2"] = bench_attn_decode(torch, 64, 32768, args.steps, args.warmup, 13)
        log("c2", res["c2"])
    if "c3" in want:
        res["c3"] = bench_attn_prefill(torch, 8192, args.steps, args.warmup, 14)
        log("c3", res["c3"])
    if "c4" in want:
        res["c4"] = bench_mixed_block(torch, 128, args.steps, args.warmup, 15)
        log("c4", res["c4"])
    for name, M, exact in (("p1", 1, True), ("p64", 64, False), ("p4096", 4096, False)):
        if name in want:
            res[name] = bench_proj(torch, M, exact, args.steps, args.warmup, 16)
            log(name, res[name])
    if "copy" in want:
        res["copy"] = bench_copy(torch, args.steps, args.warmup)
        log("copy", res["copy"])

    head = res.get("c1") or next((v for v in res.values() if "roofline" in v), None)
    if head is None:                       # calibration-only run
        print(json.dumps(dict(metric="copy calibration", configs=_rounded(res))))
        return
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_threads, args.cpu_tokens)
    roof = head["roofline"]
    line = dict(metric="attn-layer tok/s @1 GPU; decode HBM GB/s % peak; prefill MFMA TFLOP/s % peak",
                value=head["tok_s"], unit="tok/s", n_gpus=1, steps=args.steps, warmup=args.warmup,
                ms_per_step=head["ms_per_step"], higher_is_better=True, scaling="weak",
                vs_baseline=None, dtype="f32", data="synthetic (bf16 storage, fp32 arithmetic)",
                config=dict(workload=head["workload"], global_batch=1,
                            seq_len=head["tokens_per_step"], parallelism="none (1 GPU)"),
                roofline=roof, cpu_baseline=cpu,
                configs=_rounded(res))
    print(json.dumps(line))


if __name__ == "__main__":
    main()
