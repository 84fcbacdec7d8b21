"""Write tests/golden/ref_vectors.npz: input/output vectors of the
reference's own scalar anchors (c/gdn.h, c/attn.h, c/bf16.h, wired as
c/layer.h by oracle/ref_shim.c), compiled from /root/reference/c into
oracle/_ref/libapus_ref.so by `make -C oracle ref`.

Run in the build container only (the reference is not present on GPU
hosts):  python tests/golden/make_golden.py

The vectors are data -- seeded inputs and the reference's outputs -- so the
oracle and the HIP library can be checked against the reference where the
reference cannot be built or loaded. Sizes are small (the file is ~100 KB).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "apus-qwen3.6-35b-a3b_amd"),
                os.path.dirname(HERE)]

import oracle  # noqa: E402
import synth   # noqa: E402


def main():
    ref = oracle.Reference()
    rng = np.random.default_rng(20260829)
    v = {}

    # conv1d over T=9 tokens of C=37 channels, continuing a state
    C_, T = 37, 9
    v["conv_x"] = synth.normal_bf16(rng, (T, C_), 1.5)
    v["conv_w"] = synth.normal_bf16(rng, (C_, 4), 0.7)
    v["conv_state0"] = synth.normal_bf16(rng, (C_ * 3,))
    st = v["conv_state0"].copy()
    v["conv_out"] = ref.gdn_conv1d(v["conv_x"], v["conv_w"], st)
    v["conv_state1"] = st

    # decay and beta (H=13), a spread wide enough to reach the x>20 branch
    H = 13
    v["gate_a"] = synth.normal_bf16(rng, (H,), 8.0)
    v["gate_b"] = synth.normal_bf16(rng, (H,), 6.0)
    v["gate_A_log"] = rng.uniform(0.0, 2.7, H).astype(np.float32)
    v["gate_dt"] = rng.standard_normal(H).astype(np.float32)
    v["decay_g"] = ref.gdn_decay(v["gate_a"], v["gate_A_log"], v["gate_dt"])
    v["beta"] = ref.gdn_beta(v["gate_b"])

    # l2norm, 3 heads of 16, q scale
    v["l2_x"] = synth.normal_bf16(rng, (3 * 16,))
    v["l2_y"] = ref.gdn_l2norm(v["l2_x"], 3, 16, 16 ** -0.5)

    # recurrence: T=5 steps, 2 heads of 16x16
    T, H, Dk, Dv = 5, 2, 16, 16
    v["rec_S0"] = (rng.standard_normal((H, Dk, Dv)) * 0.05).astype(np.float32)
    v["rec_q"] = (rng.standard_normal((T, H, Dk)) * 0.25).astype(np.float32)
    v["rec_k"] = (rng.standard_normal((T, H, Dk)) * 0.25).astype(np.float32)
    v["rec_v"] = synth.normal_bf16(rng, (T, H, Dv))
    v["rec_g"] = (-rng.uniform(0.0, 2.0, (T, H))).astype(np.float32)
    v["rec_beta"] = synth.bf16_bits(rng.uniform(0.0, 1.0, (T, H)).astype(np.float32))
    S = v["rec_S0"].copy()
    v["rec_o"] = ref.gdn_recurrent(S, v["rec_q"], v["rec_k"], v["rec_v"], v["rec_g"],
                                   v["rec_beta"], T, H, Dk, Dv)
    v["rec_S1"] = S

    # gated RMSNorm, 3 heads of 32
    v["on_o"] = synth.normal_bf16(rng, (3 * 32,))
    v["on_z"] = synth.normal_bf16(rng, (3 * 32,))
    v["on_w"] = synth.normal_bf16(rng, (32,), 0.1, 1.0)
    v["on_y"] = ref.gdn_onorm(v["on_o"], v["on_z"], v["on_w"], 3, 32)

    # (1+w) RMSNorm, N=256; partial RoPE (rot 64) at three positions
    v["rms_x"] = synth.normal_bf16(rng, (256,))
    v["rms_w"] = synth.normal_bf16(rng, (256,), 0.1)
    v["rms_y"] = ref.attn_rmsnorm(v["rms_x"], v["rms_w"])
    v["rope_x"] = synth.normal_bf16(rng, (256,))
    v["rope_pos"] = np.array([0.0, 7.0, 32767.0], np.float32)
    v["rope_y"] = np.stack([ref.attn_rope(v["rope_x"], 64, float(p)) for p in v["rope_pos"]])

    # causal GQA: Tq=3 rows at the end of Tk=9 keys, 4 q heads / 2 kv, d=32
    Tq, Tk, H, Hkv, D = 3, 9, 4, 2, 32
    v["gqa_q"] = synth.normal_bf16(rng, (Tq, H, D))
    v["gqa_k"] = synth.normal_bf16(rng, (Tk, Hkv, D))
    v["gqa_v"] = synth.normal_bf16(rng, (Tk, Hkv, D))
    v["gqa_o"] = ref.attn_gqa(v["gqa_q"], v["gqa_k"], v["gqa_v"], Tq, Tk, H, Hkv, D,
                              float(1.0 / np.sqrt(D)))

    # output gate
    v["og_o"] = synth.normal_bf16(rng, (64,))
    v["og_gate"] = synth.normal_bf16(rng, (64,), 3.0)
    v["og_y"] = ref.attn_outgate(v["og_o"], v["og_gate"])

    # GDN mixer at reduced dims (hk=2, hv=4, dk=dv=16): 2 sequences, 3 + 2 tokens
    dims = (2, 4, 16, 16)
    w = synth.gdn_weights(rng, dims)
    for k_, a_ in w.items():
        v["gm_w_" + k_] = a_
    v["gm_cu"] = np.array([0, 3, 5], np.int32)
    tok = synth.gdn_tokens(rng, 5, dims)
    for k_, a_ in tok.items():
        v["gm_" + k_] = a_
    conv, S = synth.gdn_state(rng, 2, dims)
    v["gm_conv0"], v["gm_S0"] = conv.copy(), S.copy()
    v["gm_y"] = ref.gdn_mixer(dims, w, v["gm_cu"], tok["qkv"], tok["z"], tok["a"], tok["b"],
                              conv, S)
    v["gm_conv1"], v["gm_S1"] = conv, S

    # attention mixer at reduced dims (nh=4, nkv=2, d=64, rot=32): 2 sequences,
    # 2 new tokens at pos 3 and 1 new token at pos 10, cache of 16 positions
    adims = (4, 2, 64, 32, 1e7)
    aw = synth.attn_weights(rng, adims)
    for k_, a_ in aw.items():
        v["am_w_" + k_] = a_
    v["am_cu"] = np.array([0, 2, 3], np.int32)
    v["am_pos0"] = np.array([3, 10], np.int32)
    atok = synth.attn_tokens(rng, 3, adims)
    for k_, a_ in atok.items():
        v["am_" + k_] = a_
    maxs = 16
    kc = synth.normal_bf16(rng, (2, maxs, 2, 64))
    vc = synth.normal_bf16(rng, (2, maxs, 2, 64))
    v["am_kc0"], v["am_vc0"] = kc.copy(), vc.copy()
    v["am_y"] = ref.attn_mixer(adims, aw, v["am_cu"], v["am_pos0"], atok["qg"], atok["k"],
                               atok["v"], kc, vc, maxs * 2 * 64)
    v["am_kc1"], v["am_vc1"] = kc, vc

    # projections (c/bf16.h:285-300): the x86 hot gemm, ragged shapes and a
    # K that is not a multiple of 8 (its own seed: the vectors above are
    # unchanged by this addition)
    prng = np.random.default_rng(20260901)
    v["gemm_w"] = synth.normal_bf16(prng, (37, 120), 0.1)
    v["gemm_x"] = synth.normal_bf16(prng, (3, 120))
    v["gemm_y"] = ref.bf16_gemm(v["gemm_w"], v["gemm_x"])
    v["gemm_w2"] = synth.normal_bf16(prng, (19, 45), 0.3)
    v["gemm_x2"] = synth.normal_bf16(prng, (2, 45))
    v["gemm_y2"] = ref.bf16_gemm(v["gemm_w2"], v["gemm_x2"])

    out = os.path.join(HERE, "ref_vectors.npz")
    np.savez_compressed(out, **v)
    print(out, os.path.getsize(out), "bytes,", len(v), "arrays")


if __name__ == "__main__":
    main()
