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


def _offset_view(a, dev):
    """The rows of a at a 4-byte offset from a 16-byte aligned allocation (and a
    row stride of K + 1 floats): the kernels' scalar-load paths."""
    M, K = a.shape
    buf = torch.zeros((M, K + 1), dtype=torch.float32, device=dev)
    buf[:, 1:] = torch.from_numpy(a).to(dev)
    v = buf[:, 1:]
    assert v.data_ptr() % 16 == 4
    return v


def run(sqa, orc, dev, N, K, M, seed, gate=True, outliers=0, scale=1.0, unaligned=False):
    rng = np.random.default_rng(seed)
    w = random_q4k(rng, N, K)
    x = rng.standard_normal((M, K)).astype(np.float32) * np.float32(scale)
    if outliers:
        x[:, rng.choice(K, outliers, replace=False)] *= 8
    g = rng.standard_normal((M, K)).astype(np.float32) if gate else None
    ref = orc.out_proj(w, x, g)
    wt = torch.from_numpy(w).to(dev)
    if unaligned:
        xt = _offset_view(x, dev)
        gt = _offset_view(g, dev) if gate else None
    else:
        xt = torch.from_numpy(x).to(dev)
        gt = torch.from_numpy(g).to(dev) if gate else None
    out = sqa.out_proj(wt, xt, gt)
    torch.cuda.synchronize()
    err = rel_max(out.cpu().numpy(), ref)
    print(f"out_proj N={N} K={K} M={M} gate={gate} scale={scale} unaligned={unaligned}: max err / rms = {err:.3e}")
    return err


@pytest.mark.parametrize("M", [1, 2, 3, 4, 13, 16, 17, 64, 100, 512])
def test_out_proj_gated_n_embd_2048(sqa, orc, dev, M):
    assert run(sqa, orc, dev, 2048, 4096, M, 100 + M, outliers=8) <= TOL


@pytest.mark.parametrize("M", [1, 3, 4, 40])
def test_out_proj_without_gate(sqa, orc, dev, M):
    assert run(sqa, orc, dev, 512, 4096, M, 200 + M, gate=False) <= TOL


@pytest.mark.parametrize("N,K,M", [(48, 256, 1), (48, 256, 33), (16, 512, 7), (80, 1024, 70), (48, 1280, 65),
                                   (2064, 768, 97), (2048, 4096, 1000)])
def test_out_proj_small_and_ragged_shapes(sqa, orc, dev, N, K, M):
    # one super-block, N not a multiple of 64 or 128 (row tiles past N), K of 3
    # or 5 super-blocks (a partial group of four for the min term), token counts
    # that are not a multiple of 32
    assert run(sqa, orc, dev, N, K, M, 300 + N + M) <= TOL


@pytest.mark.parametrize("M,gate", [(3, True), (3, False), (40, True), (1, True)])
def test_out_proj_unaligned_activations(sqa, orc, dev, M, gate):
    # x and gate rows 4 bytes off 16-byte alignment: the scalar-load forms of the
    # decode kernel (M <= 4) and of the activation pass (M > 4)
    assert run(sqa, orc, dev, 1024, 4096, M, 400 + M, gate=gate, unaligned=True) <= TOL


@pytest.mark.parametrize("M,scale", [(1, 1e-4), (1, 3e3), (4, 1e-4), (4, 3e3), (17, 1e-2), (17, 1e3),
                                     (512, 1e-2), (512, 1e3)])
def test_out_proj_activation_scale(sqa, orc, dev, M, scale):
    # up to 4 tokens the activations stay fp32 (any size); above, the fp16 hi + lo
    # pair holds 1e-4 x RMS for activation RMS from 1e-2 up to 32-value sums
    # below 65504 (1e3 x N(0,1) with 8x outlier channels)
    assert run(sqa, orc, dev, 1024, 4096, M, 500 + M, outliers=8, scale=scale) <= TOL


def test_out_proj_large_ubatch_without_gate(sqa, orc, dev):
    assert run(sqa, orc, dev, 512, 4096, 2048, 17, gate=False) <= TOL


def test_out_proj_rejects_unsupported_shapes(sqa, dev):
    w = torch.zeros((40, 144), dtype=torch.uint8, device=dev)  # N = 40: not a multiple of 16
    x = torch.zeros((1, 256), device=dev)
    with pytest.raises(sqa.SqaError):
        sqa.out_proj(w, x)
