import numpy as np

from ds4cuda_amd import synth


def test_splitmix64_published_vector():
    # splitmix64 with state 0: first outputs of the reference algorithm
    z = synth.splitmix64(0, 3)
    assert [int(v) for v in z] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_normal_is_deterministic_and_standard():
    a = synth.normal(0, 1, 200001)
    b = synth.normal(0, 1, 200001)
    assert np.array_equal(a, b) and a.dtype == np.float32
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1) < 0.01
    assert not np.array_equal(a[:1000], synth.normal(0, 2, 1000))


def test_bf16_rounding():
    x = np.float32([1.0, 1.00390625, 1.005859375, -3.0e-3, 65504.0])
    h = synth.to_bf16_bits(x)
    back = synth.bf16_bits_to_f32(h)
    assert back[0] == 1.0 and back[1] == 1.0          # tie to even
    assert back[2] == np.float32(1.0078125)
    assert np.all(np.abs(back - x) <= np.abs(x) * 2.0 ** -8)


def test_outlier_rows():
    x = synth.kv_rows(0, 3, 4000, 64, outlier_frac=0.01)
    big = np.abs(x).max(axis=1) > 6.0
    assert 10 <= big.sum() <= 90


def test_device_generator_matches_host():
    # the torch form (run here on the CPU device) gives the host stream exactly
    from ds4cuda_amd import synth
    a = synth.normal(3, 5, 100001)
    b = synth.normal_device(3, 5, 100001, "cpu", chunk=30000).numpy()
    assert np.array_equal(a, b)
    a = synth.kv_rows(7, 2, 300, outlier_frac=0.05)
    b = synth.kv_rows_device(7, 2, 300, "cpu", outlier_frac=0.05).numpy()
    assert np.array_equal(a, b)
