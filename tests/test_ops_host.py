"""The Python mirror refuses host tensors for device buffers (the kernels
would read host memory and fault the GPU) and wrong dtypes or sizes, with
Ds4HipError(-22), before any device work: no GPU needed."""
import pytest
import torch

from ds4cuda_amd import Ds4HipError, ops


def refused(fn, *args, **kw):
    with pytest.raises(Ds4HipError) as e:
        fn(*args, **kw)
    assert e.value.code == -22
    return str(e.value)


def test_host_tensors_are_refused():
    x = torch.zeros(4 * 512)
    msg = refused(ops.launch_fp8_kv_quantize_round_trip_f32, x, x, 4, 512, 64)
    assert "GPU tensor" in msg
    refused(ops.launch_rms_norm_f32, torch.zeros(16), torch.zeros(16), torch.zeros(16), 16)
    q = torch.zeros(64 * 512)
    refused(ops.launch_flash_attn_decode_mixed_f32, q, torch.zeros(512), None, None, torch.zeros(64), q,
            64, 1, 0, 512)


def test_meta_tensors_are_refused():
    # device-independent: a tensor with no storage on the GPU is refused the same way
    x = torch.empty(4 * 512, device="meta")
    refused(ops.launch_fp8_kv_quantize_round_trip_f32, x, x, 4, 512, 64)
