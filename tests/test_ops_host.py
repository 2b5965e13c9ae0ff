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


class FakeGpu:
    """Stands in for a GPU tensor in the argument checks (never reaches a kernel:
    every call below is refused on another argument first)."""

    def __init__(self, numel, dtype=torch.float32):
        self._n, self.dtype = numel, dtype
        self.device = torch.device("cuda", 0) if torch.cuda.is_available() else type("D", (), {"type": "cuda"})()

    def numel(self):
        return self._n

    def element_size(self):
        return torch.empty(0, dtype=self.dtype).element_size()

    def is_contiguous(self):
        return True

    def data_ptr(self):
        return 0


def test_host_buffers_refused_in_every_slot():
    """sinks, out, workspaces and scratch buffers are checked like the inputs."""
    n = 64 * 512
    g = FakeGpu
    host = torch.zeros(n)
    msg = refused(ops.launch_flash_attn_decode_mixed_f32, g(n), g(512), None, None, host, g(n), 64, 1, 0, 512)
    assert "sinks" in msg
    msg = refused(ops.launch_flash_attn_decode_mixed_f32, g(n), g(512), None, None, g(64), host, 64, 1, 0, 512)
    assert "out" in msg
    msg = refused(ops.launch_flash_attn_decode_mixed_f32_prealloc, g(n), g(512), None, None, g(64), g(n), 64, 1,
                  0, 512, torch.zeros(100, dtype=torch.uint8))
    assert "workspace" in msg
    msg = refused(ops.launch_flash_attn_decode_raw_f32_prealloc, g(n), g(512), g(512), g(64), g(n), 64, 1, 512,
                  torch.zeros(100, dtype=torch.uint8))
    assert "workspace" in msg
    W = g(4096 * 256 * 34, torch.uint8)
    msg = refused(ops.launch_mul_mv_q8_0_q8_0_f32_prealloc, W, g(8192), g(4096), 4096, 8192,
                  torch.zeros(8192, dtype=torch.int8), g(256))
    assert "scratch_xq" in msg
    msg = refused(ops.launch_mul_mv_q8_0_q8_0_f32_prealloc, W, host, g(4096), 4096, 8192, g(8192, torch.int8),
                  g(256))
    assert "x" in msg
    msg = refused(ops.launch_indexer_score_topk_f32_i32, g(64 * 128), g(64), g(1000 * 128), 1000, 64, 128, 512,
                  torch.zeros(1000, dtype=torch.int32), g(1000))
    assert "allowed_out" in msg
    msg = refused(ops.launch_compressor_decode_step_f32_prealloc, 1, g(4096), g(1), g(1), g(1), g(512), 4096, 512,
                  4, 0, 2, g(1), g(1), g(512), torch.zeros(1024), g(1024))
    assert "scratch_kv_cur" in msg
