"""The W_o projection on the GPU against the oracle (reference: the gate and
ggml_mul_mat(attn_output, gated) of src/model/attn.rs:281-285).

The oracle is an fp64 GEMM over ggml's fp32 dequantized Q4_K weights and the
fp32 gated activations. Tolerance: max |gpu - oracle| <= 1e-4 x RMS(oracle):
the kernel multiplies the exact codes by the activations held to ~22 bits and
accumulates in fp32. (ggml's CPU path rounds the activations to 8 bits; its
results sit about 1e-2 x RMS from the same fp64 value, which is why the
reference's own test, tests/kernel_verify.rs:553-590, compares against an f32
matmul with a quantization bound.)"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
TOL = 1e-4


def random_q4k(rng, n, k):
    """Q4_K rows with random codes and 6-bit (scale, min) pairs and positive fp16 d, dmin
    of the size real weights have."""
    w = rng.integers(0, 256, (n, k // 256, 144), dtype=np.uint8)
    d = rng.uniform(2e-4, 4e-3, (n, k // 256)).astype(np.float16)
    dmin = rng.uniform(0, 4e-3, (n, k // 256)).astype(np.float16)
    w[:, :, 0:2] = d.view(np.uint8).reshape(n, k // 256, 2)
    w[:, :, 2:4] = dmin.view(np.uint8).reshape(n, k // 256, 2)
    return w.reshape(n, k // 256 * 144)


def rel_max(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / np.sqrt(np.mean(ref ** 2)))


def run(sqa, orc, dev, N, K, M, seed, gate=True, outliers=0):
    rng = np.random.default_rng(seed)
    w = random_q4k(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    if outliers:
        x[:, rng.choice(K, outliers, replace=False)] *= 8
    g = rng.standard_normal((M, K)).astype(np.float32) if gate else None
    ref = orc.out_proj(w, x, g)
    wt = torch.from_numpy(w).to(dev)
    xt = torch.from_numpy(x).to(dev)
    gt = torch.from_numpy(g).to(dev) if gate else None
    out = sqa.out_proj(wt, xt, gt)
    torch.cuda.synchronize()
    err = rel_max(out.cpu().numpy(), ref)
    print(f"out_proj N={N} K={K} M={M} gate={gate}: max err / rms = {err:.3e}")
    return err


@pytest.mark.parametrize("M", [1, 2, 13, 16, 17, 64, 100, 512])
def test_out_proj_gated_n_embd_2048(sqa, orc, dev, M):
    assert run(sqa, orc, dev, 2048, 4096, M, 100 + M, outliers=8) <= TOL


@pytest.mark.parametrize("M", [1, 40])
def test_out_proj_without_gate(sqa, orc, dev, M):
    assert run(sqa, orc, dev, 512, 4096, M, 200 + M, gate=False) <= TOL


@pytest.mark.parametrize("N,K,M", [(48, 256, 1), (48, 256, 33), (16, 512, 7), (80, 1024, 70), (48, 1280, 65),
                                   (2064, 768, 97), (2048, 4096, 1000)])
def test_out_proj_small_and_ragged_shapes(sqa, orc, dev, N, K, M):
    # one super-block, N not a multiple of 64 or 128 (row tiles past N), K of 3
    # or 5 super-blocks (a partial group of four for the min term), token counts
    # that are not a multiple of 32
    assert run(sqa, orc, dev, N, K, M, 300 + N + M) <= TOL


def test_out_proj_large_ubatch_without_gate(sqa, orc, dev):
    assert run(sqa, orc, dev, 512, 4096, 2048, 17, gate=False) <= TOL


def test_out_proj_rejects_unsupported_shapes(sqa, dev):
    w = torch.zeros((40, 144), dtype=torch.uint8, device=dev)  # N = 40: not a multiple of 16
    x = torch.zeros((1, 256), device=dev)
    with pytest.raises(sqa.SqaError):
        sqa.out_proj(w, x)
