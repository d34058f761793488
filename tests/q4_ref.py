"""Independent numpy restatement of ggml's q4_0 block rule, used by the tests
to cross-check the C oracle on many random blocks. Every product and sum is a
separately rounded float32 operation, the semantics of ggml's scalar
quantize_row_q4_0_ref (rules restated in the reference at
tests/attn_test.rs:781-788: d = max/-8, codes cover [-8d, 7d])."""
import numpy as np


def quantize_blocks_np(x):
    """x float32 (nblocks, 32) -> (d_fp16_bits uint16 (nblocks,), codes uint8 (nblocks, 32))."""
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x)
    amax = a.max(axis=1)
    first = np.argmax(a == amax[:, None], axis=1)  # first index attaining the maximum
    mx = x[np.arange(x.shape[0]), first]
    mx = np.where(amax == 0, np.float32(0.0), mx).astype(np.float32)
    d = (mx / np.float32(-8.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, np.float32(1.0)), np.float32(0.0)).astype(np.float32)
    prod = (x * idv[:, None]).astype(np.float32)
    y = (prod + np.float32(8.5)).astype(np.float32)
    codes = np.minimum(np.trunc(y).astype(np.int32), 15).astype(np.uint8)
    return d.astype(np.float16).view(np.uint16), codes


def pack_blocks(dbits, codes):
    """(d bits, codes) -> q4_0 bytes (nblocks, 18): qs[j] = c[j] | c[j+16] << 4."""
    nb = codes.shape[0]
    out = np.zeros((nb, 18), dtype=np.uint8)
    out[:, 0] = dbits & 0xFF
    out[:, 1] = dbits >> 8
    out[:, 2:] = codes[:, :16] | (codes[:, 16:] << 4)
    return out
