"""The committed fixtures under tests/golden/ (written by make_golden.py from
the oracle) against (1) the oracle itself, re-run now, bit for bit, and
(2) independent checks: the numpy restatement of the q4_0 rule for the
quantizer blocks, and fp64 brute-force attention on the dequantized operands
for the attention cases."""
import os

import numpy as np
import pytest

from tests import fa_ref, q4_ref

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FA_CASES = ["fa_decode_outliers", "fa_verify_causal", "fa_prefill_gate", "fa_prefill_g4"]


def load(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"))


def test_q4_0_blocks_oracle_and_numpy(orc):
    g = load("q4_0_blocks")
    x, want = g["x"], g["q4_0"]
    got = orc.quantize_q4_0(x.reshape(1, -1)).reshape(want.shape)
    assert np.array_equal(got, want)
    d, codes = q4_ref.quantize_blocks_np(x)
    assert np.array_equal(q4_ref.pack_blocks(d, codes), want)
    # closed forms: the all-zero block is d = -0.0 with every byte 0x88; the
    # ramp j - 16 has max -16, d = 2, and element 0 (the max) gets code 0
    assert want[0, 0] == 0x00 and want[0, 1] == 0x80 and np.all(want[0, 2:] == 0x88)
    assert want[1, :2].view(np.float16)[0] == np.float16(2.0) and (want[1, 2] & 15) == 0


@pytest.mark.parametrize("name", FA_CASES)
def test_fa_fixture_matches_oracle(orc, name):
    g = load(name)
    out = orc.flash_attn_ext(g["q"], g["k"], g["v"], g["mask"], scale=float(g["scale"]))
    if "gate" in g:
        n_q = out.shape[0]
        out = orc.sigmoid_mul(out.reshape(n_q, -1), g["gate"].reshape(n_q, -1)).reshape(out.shape)
    assert np.array_equal(out, g["out"])


@pytest.mark.parametrize("name", FA_CASES)
def test_fa_fixture_against_f64_brute_force(orc, name):
    g = load(name)
    qd = fa_ref.q8_dequant(orc, g["q"])
    kd = fa_ref.cache_dequant(orc, g["k"])
    vd = fa_ref.cache_dequant(orc, g["v"])
    ref = fa_ref.attention_f64(qd, kd, vd, float(g["scale"]), g["mask"])
    if "gate" in g:
        ref = ref / (1.0 + np.exp(-g["gate"].astype(np.float64)))
    assert fa_ref.rel_err(g["out"], ref) < 1e-5
