"""The fp8 oracle (no reference counterpart): e4m3 rounding and the dequantized-operand formula.

Pins: an exhaustive nearest-value search over the 254 finite e4m3 values
(ties to even mantissa) against torch's float8_e4m3fn cast; a closed form for
constant inputs, where every slot sum is the slot's neighbour count and counts
above 16 must round to the e4m3 grid (17 -> 16, 19 -> 20, ...); equality with
the fp32 oracle on dequantized operands for single-neighbour slots.
"""
import numpy as np
import torch

from oracle import knnconv_ref
from tests.helpers import layer_tables


def test_e4m3_value_table():
    v = knnconv_ref.e4m3_values()
    assert np.isnan(v[0x7F]) and np.isnan(v[0xFF]) and np.isnan(v).sum() == 2
    assert v[0x7E] == 448.0 and v[0x01] == 2.0 ** -9 and v[0x08] == 2.0 ** -6 and v[0x38] == 1.0
    finite = v[~np.isnan(v)]
    assert len(np.unique(finite)) == 253      # +0 and -0 coincide


def test_torch_cast_is_round_to_nearest_even():
    rng = np.random.default_rng(0)
    grid = knnconv_ref.e4m3_values()
    grid = grid[~np.isnan(grid) & (grid > 0)]
    mids = (grid[1:] + grid[:-1]) / 2                      # exact ties
    x = np.concatenate([rng.standard_normal(4000) * 40, rng.standard_normal(2000) * 0.02, mids, -mids,
                        np.nextafter(mids, 0), np.nextafter(mids, 1e9), [0.0, 448.0, 2.0 ** -10, 2.0 ** -11]])
    x = x.astype(np.float32).astype(np.float64)           # inputs exactly representable in fp32
    want = knnconv_ref.e4m3_round_bruteforce(x)
    got = torch.from_numpy(x).float().to(torch.float8_e4m3fn).double().numpy()
    np.testing.assert_array_equal(got, want)
    got_q = knnconv_ref.quantize_e4m3(torch.from_numpy(x).float() * 2, torch.tensor(2.0)).double().numpy()
    np.testing.assert_array_equal(got_q, want)


def _fp8_case(seed=0):
    t = layer_tables(32, 16, 25)
    g = torch.Generator().manual_seed(seed)
    c, c_out = 4, 6
    wq = knnconv_ref.quantize_e4m3(torch.randn(c_out, c * t["V"], generator=g), torch.tensor(1 / 64))
    return t, c, c_out, wq, g


def test_fp8_oracle_constant_input_closed_form():
    t, c, c_out, wq, g = _fp8_case()
    cnt = t["rf"].sum(1)                                       # [N_out, V] neighbour counts
    assert int(cnt.max()) > 16, "the case must contain slot sums beyond the exact e4m3 integers"
    xq = torch.ones(1, c, t["n_in"])
    w_scale = torch.rand(c_out, generator=g) + 0.5
    y = knnconv_ref.knnconv_fp8_forward(xq, 0.25, t["idx"], t["n_in"], t["rf"], wq, w_scale)
    r = torch.from_numpy(knnconv_ref.e4m3_round_bruteforce(cnt.double().numpy()))   # round(count)
    r = torch.where(cnt >= 2, r, cnt.double())
    wsum = wq.double().reshape(c_out, c, -1).sum(1)            # [C_out, V]
    want = 0.25 * w_scale.double()[:, None] * (wsum @ r.T)     # [C_out, N_out]
    torch.testing.assert_close(y[0], want, rtol=1e-12, atol=1e-12)
    assert not torch.equal(r, cnt.double()), "rounding of large counts must change the sum"


def test_fp8_oracle_equals_fp32_oracle_on_single_slots():
    t, c, c_out, wq, g = _fp8_case(1)
    rf = t["rf"].clone()
    # keep only the first neighbour of each multi-neighbour slot: every slot has <= 1 neighbour
    first = (rf.cumsum(1) == 1) & (rf > 0)
    rf = rf * first
    assert int(rf.sum(1).max()) == 1
    xq = knnconv_ref.quantize_e4m3(torch.randn(2, c, t["n_in"], generator=g), torch.tensor(1 / 32))
    w_scale = torch.rand(c_out, generator=g) + 0.5
    bias = torch.randn(c_out, generator=g)
    y = knnconv_ref.knnconv_fp8_forward(xq, 0.5, t["idx"], t["n_in"], rf, wq, w_scale, bias)
    w_eff = wq.double() * w_scale.double()[:, None] * 0.5
    ref = knnconv_ref.knnconv_forward(xq.double(), t["idx"], t["n_in"], rf.double(), w_eff.double(),
                                      bias.double())
    torch.testing.assert_close(y, ref, rtol=1e-12, atol=1e-10)
