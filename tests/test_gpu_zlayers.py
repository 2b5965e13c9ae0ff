"""All 43 layers of the cfg 2 decode step (43 x 32768 FP8 rows, bf16 Q, one
multi-problem launch): the default kernel against the register-load kernel
with hi + lo P (exact_p), layer by layer, at the decode
bar, plus the middle layer against the CPU oracle. The full-size parity test
checks only the first and last layer against the oracle; workgroup chunks
that straddle the other 41 layer boundaries are covered here."""
import numpy as np
import pytest
import torch

import oracle as O
from ds4cuda_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu

TOL = 2e-3


def test_cfg2_all_layers_two_kernels(gpu):
    n_layer, n_kv = 43, 32768
    cache = ops.Fp8KVCache.empty(n_layer * n_kv, device=gpu)
    for l in range(n_layer):
        cache.append(synth.kv_rows_device(71, l, n_kv, gpu, outlier_frac=0.01), row0=l * n_kv)
    bits = synth.to_bf16_bits(synth.normal(72, 0, n_layer * 64 * 512)).reshape(n_layer, 64, 512)
    q = torch.from_numpy(bits.view(np.int16)).to(gpu).view(torch.bfloat16)
    sinks_h = synth.normal(72, 1, n_layer * 64).reshape(n_layer, 64).astype(np.float32)
    sinks = torch.from_numpy(sinks_h).to(gpu)
    outs = []
    for exact in (0, 1):
        out = torch.zeros((n_layer, 64, 512), dtype=torch.float32, device=gpu)
        ops.flash_attn_decode_fp8(q, sinks, out, cache, [n_kv] * n_layer, row_base_stride=n_kv,
                                  exact_p=bool(exact))
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy().astype(np.float64))
    worst = 0.0
    for l in range(n_layer):
        ref = outs[1][l]
        rms = np.sqrt(np.mean(ref ** 2))
        err = np.abs(outs[0][l] - ref).max() / rms
        worst = max(worst, err)
        assert np.isfinite(outs[0][l]).all() and err <= TOL, (l, err)
    # the middle layer against the oracle
    l = 21
    codes = cache.codes.cpu().numpy()
    sexp = cache.sexp.cpu().numpy()
    tail = cache.tail.cpu().numpy().view(np.uint16)
    qf = synth.bf16_bits_to_f32(bits[l])
    ref = O.attn_decode_fp8(qf, codes, sexp, tail, l * n_kv + np.arange(n_kv), sinks_h[l], n_threads=8)
    err = np.abs(outs[0][l] - ref).max() / np.sqrt(np.mean(ref.astype(np.float64) ** 2))
    print(f"43 layers: worst err/RMS between the kernels {worst:.2e}; layer 21 vs oracle {err:.2e}")
    assert err <= TOL
