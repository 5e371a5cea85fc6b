"""Host-side logic without a GPU: block layouts, synthetic generators, bf16
rounding."""
import numpy as np

from realm_amd import formats, synth


def test_block_sizes():
    assert formats.Q4K_DTYPE.itemsize == 144
    assert formats.Q6K_DTYPE.itemsize == 210
    assert formats.Q80_DTYPE.itemsize == 34
    assert formats.weight_bytes(formats.GGML_Q4_K, 5632, 2048) == 6_488_064
    assert formats.weight_bytes(formats.GGML_Q6_K, 4096, 11008) == 36_986_880
    assert formats.weight_bytes(formats.GGML_Q8_0, 11008, 4096) == 47_906_816


def test_generators_are_seeded_and_in_range():
    a = synth.q4k_blocks(synth.rng(1), 16, 512)
    b = synth.q4k_blocks(synth.rng(1), 16, 512)
    assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
    d = a["d"].view(np.float16).astype(np.float64)
    assert np.all(d >= 0) and 3e-4 < d.mean() < 1.3e-3  # |N(0,1)|*1e-3: mean 0.8e-3
    s6 = synth.q6k_blocks(synth.rng(2), 64, 512)
    assert s6["scales"].min() >= -32 and s6["scales"].max() <= 31
    q8 = synth.q80_blocks(synth.rng(3), 64, 256)
    assert q8["quants"].min() >= -127 and q8["quants"].max() <= 127


def test_bf16_round_trip():
    g = np.random.default_rng(0)
    x = g.standard_normal(10000).astype(np.float32)
    b = synth.f32_to_bf16_bits(x)
    y = synth.bf16_bits_to_f32(b)
    assert np.all(np.abs(y - x) <= np.abs(x) * 2.0 ** -8)
    # exact for values already in bf16
    assert np.array_equal(synth.f32_to_bf16_bits(y), b)
    # ties to even
    t = np.array([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8], np.float32)
    assert np.array_equal(synth.bf16_bits_to_f32(synth.f32_to_bf16_bits(t)),
                          np.array([1.0, 1.0 + 2.0 ** -6], np.float32))


def test_adapter_ids_distribution():
    ids = synth.adapter_ids(synth.rng(4), 20000, 16)
    assert ids.min() == -1 and ids.max() == 15
    assert abs((ids == -1).mean() - 0.1) < 0.01
    counts = np.bincount(ids[ids >= 0], minlength=16)
    assert counts[0] > counts[1] > counts[4] > counts[15]  # Zipf: decreasing
