"""CPU pinning of oracle/numerics.py: bf16 conversions against torch's own cast."""
import numpy as np
import torch

from oracle.numerics import bf16_bits_to_f32, f32_to_bf16_bits, softplus


def test_bf16_round_trip_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100000) * 10, rng.standard_normal(1000) * 1e-30,
                        [0.0, -0.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 3.4e38, -3.4e38, np.inf,
                         -np.inf]]).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(f32_to_bf16_bits(x), ref)
    back = torch.from_numpy(ref.view(np.int16)).view(torch.bfloat16).float().numpy()
    assert np.array_equal(bf16_bits_to_f32(ref), back)


def test_bf16_nan_stays_nan():
    x = np.array([np.nan, -np.nan], np.float32)
    assert np.isnan(bf16_bits_to_f32(f32_to_bf16_bits(x))).all()


def test_softplus_matches_torch():
    x = np.linspace(-30, 30, 1001)
    np.testing.assert_allclose(softplus(x), torch.nn.functional.softplus(torch.from_numpy(x)).numpy(),
                               rtol=1e-12, atol=1e-300)
