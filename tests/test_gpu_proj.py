"""GPU parity: the projections on either side of the path (c/bf16.h:
178-231) through the C ABI against the oracle (itself bitwise the
reference's x86 hot path, tests/test_oracle_ref.py).

The hook drop-ins (host pointers) and the device-pointer sequential kernel
keep the reference's order and must be bitwise. The MFMA GEMM (hand-written,
every row count) sums in the MFMA's order: every element within 2e-3 (|r| + esc), esc = sum_k |w x|
(the attention kernels' class), and normwise within 2e-3.
"""
import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu

SHAPES = [(1, 12352, 2048),     # GDN in_proj (qkv | z | a | b) at one token
          (3, 2048, 4096),      # GDN out_proj, three tokens
          (2, 517, 40),         # ragged outputs, a short K
          (1, 33, 37)]          # K not a multiple of 8 (the scalar path)


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to("cuda")


@pytest.mark.parametrize("M,O,K", SHAPES)
def test_gemm_hooks_bitwise(hip, orc, M, O, K):
    rng = np.random.default_rng(M * 1000003 + O * 7 + K)
    w = synth.normal_bf16(rng, (O, K), K ** -0.5)
    x = synth.normal_bf16(rng, (M, K))
    print(f"[proj] hooks M={M} O={O} K={K}", flush=True)
    y = hip.bf16_gemm(w, x)
    r = orc.bf16_gemm(w, x)
    assert np.array_equal(y, r)
    assert np.array_equal(hip.bf16_gemv(w, np.ascontiguousarray(x[0])), r[0])


def test_gemm_hooks_weight_copies(hip, orc):
    """Weights are copied once per host buffer: repeated calls reuse the
    copy; another buffer (or a released cache) gets its own."""
    rng = np.random.default_rng(5)
    w1 = synth.normal_bf16(rng, (300, 256), 0.1)
    w2 = synth.normal_bf16(rng, (300, 256), 0.1)
    x = synth.normal_bf16(rng, (2, 256))
    for _ in range(2):
        assert np.array_equal(hip.bf16_gemm(w1, x), orc.bf16_gemm(w1, x))
        assert np.array_equal(hip.bf16_gemm(w2, x), orc.bf16_gemm(w2, x))
    hip.bf16_weights_release()
    w1[:] = w2
    assert np.array_equal(hip.bf16_gemm(w1, x), orc.bf16_gemm(w2, x))


@pytest.mark.parametrize("M,O,K", SHAPES)
def test_gemm_dev_bitwise(hip, orc, M, O, K):
    import torch
    rng = np.random.default_rng(M + O + K)
    w = synth.normal_bf16(rng, (O, K), K ** -0.5)
    x = synth.normal_bf16(rng, (M, K))
    y = torch.empty((M, O), dtype=torch.int16, device="cuda")
    hip.bf16_gemm_dev(_dev(torch, w), _dev(torch, x), y, exact=True)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint16), orc.bf16_gemm(w, x))


def test_gemm_dev_bitwise_wide_range(hip, orc):
    """Operands whose magnitudes span 2^-60 .. 2^60 (every product still in
    fp32's normal range): the sequential kernel's fused multiply-add rounds
    where the reference's multiply-then-add does, so the result stays
    bitwise; exact zeros and sign mixes included."""
    import torch
    rng = np.random.default_rng(77)
    O, K, M = 4096, 2048, 2
    def wide(shape):
        v = rng.standard_normal(shape) * np.exp2(rng.integers(-60, 61, shape))
        v[rng.random(shape) < 0.05] = 0.0
        return synth.bf16_bits(v.astype(np.float32))
    w, x = wide((O, K)), wide((M, K))
    y = torch.empty((M, O), dtype=torch.int16, device="cuda")
    hip.bf16_gemm_dev(_dev(torch, w), _dev(torch, x), y, exact=True)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint16), orc.bf16_gemm(w, x))
    assert np.array_equal(hip.bf16_gemv(w, np.ascontiguousarray(x[0])), orc.bf16_gemm(w, x)[0])


# one shape per tile configuration of the MFMA GEMM (64 x 64, 128 x 128,
# 128 x 256, 256 x 256), with ragged row / output edges and an output count
# that is not a multiple of 4 (the element-store epilogue)
@pytest.mark.parametrize("M,O,K", [(64, 12352, 2048), (200, 1000, 4096), (1, 70, 32),
                                   (300, 5000, 512),    # 128 x 128 tiles
                                   (260, 10240, 256),   # 128 x 256 tiles
                                   (1000, 1000, 512),   # 256 x 256, ragged edges
                                   (700, 517, 64)])     # O % 4 != 0
def test_gemm_mfma_tolerance(hip, orc, M, O, K):
    import torch
    rng = np.random.default_rng(M * 31 + K)
    w = synth.normal_bf16(rng, (O, K), K ** -0.5)
    x = synth.normal_bf16(rng, (M, K))
    print(f"[proj] mfma M={M} O={O} K={K}", flush=True)
    y = torch.empty((M, O), dtype=torch.int16, device="cuda")
    hip.bf16_gemm_dev(_dev(torch, w), _dev(torch, x), y, exact=False)
    torch.cuda.synchronize()
    c = synth.bf16_f32(y.cpu().numpy().view(np.uint16)).astype(np.float64)
    r = synth.bf16_f32(orc.bf16_gemm(w, x)).astype(np.float64)
    esc = np.abs(synth.bf16_f32(x).astype(np.float64)) @ np.abs(synth.bf16_f32(w).astype(np.float64)).T
    assert np.all(np.abs(c - r) <= 2e-3 * (np.abs(r) + esc))
    nrm = np.linalg.norm(c - r) / np.linalg.norm(r)
    same = float(np.mean(c == r))
    print(f"[proj] mfma normwise {nrm:.3g}, identical {same:.4f}", flush=True)
    assert nrm <= 2e-3 and same > 0.9


def test_gemm_mfma_refuses_unaligned_k(hip):
    """K not a multiple of 32: the MFMA GEMM returns "unsupported" (the
    caller runs the exact kernel or its CPU op), never a wrong result."""
    import torch
    w = torch.zeros((90, 40), dtype=torch.int16, device="cuda")
    x = torch.zeros((7, 40), dtype=torch.int16, device="cuda")
    y = torch.empty((7, 90), dtype=torch.int16, device="cuda")
    with pytest.raises(hip.ApusHipError) as e:
        hip.bf16_gemm_dev(w, x, y, exact=False)
    assert e.value.code == 1
