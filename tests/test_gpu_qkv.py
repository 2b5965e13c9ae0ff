"""The decode Q / KV producer (Steps 3-10 of cuda/forward_layer.cu:827-913)
and the RMSNorm launchers (cuda/norm.cuh:24,40) on the GPU, against the CPU
oracle:

  * RMSNorm, single row and the three batch weight modes: 1e-5 x RMS (fp32
    accumulation in another order than the oracle's fp64);
  * ds4hip_attn_qkv_decode_f32 piece by piece, each piece from the device's
    own input (the Q8_0 activation rounding is discontinuous): q_lora_norm
    from attn_norm, q_cur from the device's q_lora_norm, kv_rope from
    attn_norm, all at 1e-5 x RMS; Steps 8-10 also against fp64 closed forms
    of the per-head norm at pos 0 (where the RoPE is the identity);
  * Step 11: the FP8 round trip of the device's kv_rope against the oracle's
    FP8 row of the oracle's kv_rope: bit-exact except at rounding midpoints.
"""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle as O
from fp8_check import check_fp8_emit
from oracle import P
from ds4cuda_amd import ops, synth
from test_oracle_misc import q8_pack, rope

pytestmark = pytest.mark.gpu


def rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / (np.sqrt(np.mean(ref ** 2)) + 1e-30))


def orc_norm(x, w, eps=1e-6):
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros_like(x)
    O.lib().orc_rms_norm_f32(P(x), P(np.ascontiguousarray(w, np.float32)) if w is not None else None,
                             P(y), C.c_int(x.size), C.c_float(eps))
    return y


def orc_q8(Wq, x, n_rows, n_cols):
    y = np.zeros(n_rows, np.float32)
    O.lib().orc_q8_matvec(P(np.ascontiguousarray(Wq)), P(np.ascontiguousarray(x, np.float32)), P(y),
                          C.c_int(n_rows), C.c_int(n_cols))
    return y


def test_rms_norm_launchers(gpu):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(4096) * 3).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(4096)).astype(np.float32)
    y = torch.empty(4096, device=gpu)
    ops.launch_rms_norm_f32(torch.from_numpy(x).to(gpu), torch.from_numpy(w).to(gpu), y, 4096)
    torch.cuda.synchronize()
    assert rel(y.cpu().numpy(), orc_norm(x, w)) < 1e-5
    rows, n = 64, 512
    xb = (rng.standard_normal((rows, n)) * rng.uniform(0.1, 10, (rows, 1))).astype(np.float32)
    for wd in (0, n, rows * n):
        wb = (1 + 0.1 * rng.standard_normal(max(wd, 1))).astype(np.float32)
        yb = torch.empty(rows * n, device=gpu)
        ops.launch_rms_norm_batch_f32(torch.from_numpy(xb).to(gpu), torch.from_numpy(wb).to(gpu),
                                      wd, yb, rows, n)
        torch.cuda.synchronize()
        got = yb.cpu().numpy().reshape(rows, n)
        ref = np.zeros_like(xb)
        O.lib().orc_rms_norm_batch_f32(P(xb), P(wb) if wd else None, C.c_int(wd), P(ref),
                                       C.c_int(rows), C.c_int(n), C.c_float(1e-6))
        assert rel(got, ref) < 1e-5, wd


@pytest.fixture(scope="module")
def qkv_weights():
    g = lambda s, n: synth.normal(120, s, n)
    w = {}
    w["q_a"], _, _ = q8_pack(g(1, 1024 * 4096).reshape(1024, 4096) * 0.02)
    w["kv_a"], _, _ = q8_pack(g(2, 512 * 4096).reshape(512, 4096) * 0.02)
    w["q_b"], _, _ = q8_pack(g(3, 32768 * 1024).reshape(32768, 1024) * 0.03)
    w["q_a_norm"] = (1 + 0.1 * g(4, 1024)).astype(np.float32)
    w["kv_a_norm"] = (1 + 0.1 * g(5, 512)).astype(np.float32)
    return w


@pytest.mark.parametrize("il,pos", [(0, 0), (0, 4097), (2, 77), (3, 70000)])
def test_attn_qkv_decode(gpu, qkv_weights, il, pos):
    W = qkv_weights
    attn_norm = synth.normal(121, pos, 4096)
    dev = {k: torch.from_numpy(np.ascontiguousarray(v)).to(gpu) for k, v in W.items()}
    q_lora_norm = torch.empty(1024, device=gpu)
    q_cur = torch.empty(64 * 512, device=gpu)
    kv_rope = torch.empty(512, device=gpu)
    ops.attn_qkv_decode_f32(torch.from_numpy(attn_norm).to(gpu), dev["q_a"], dev["q_a_norm"],
                            dev["kv_a"], dev["kv_a_norm"], dev["q_b"], pos, il, q_lora_norm, q_cur,
                            kv_rope)
    kv_fp8 = torch.empty(512, device=gpu)
    ops.launch_fp8_kv_quantize_round_trip_f32(kv_rope, kv_fp8, 1, 512, 64)
    torch.cuda.synchronize()
    qln, qc, kvr = q_lora_norm.cpu().numpy(), q_cur.cpu().numpy(), kv_rope.cpu().numpy()
    # Steps 3-4
    ref_qln = orc_norm(orc_q8(W["q_a"], attn_norm, 1024, 4096), W["q_a_norm"])
    assert rel(qln, ref_qln) < 1e-5
    # Steps 7-9 from the device's q_lora_norm
    q_raw = orc_q8(W["q_b"], qln, 32768, 1024).reshape(64, 512)
    q_norm = np.zeros_like(q_raw)
    O.lib().orc_rms_norm_batch_f32(P(q_raw), None, C.c_int(0), P(q_norm), C.c_int(64), C.c_int(512),
                                   C.c_float(1e-6))
    ref_qc = rope(q_norm, pos, il)
    assert rel(qc, ref_qc.reshape(-1)) < 1e-5
    if pos == 0:   # RoPE is the identity: per-head unit-RMS rows (fp64 closed form)
        q64 = q_raw.astype(np.float64)
        closed = q64 / np.sqrt((q64 ** 2).mean(axis=1, keepdims=True) + 1e-6)
        assert rel(qc, closed.reshape(-1)) < 1e-5
    # Steps 5, 6, 10
    kv_raw = orc_q8(W["kv_a"], attn_norm, 512, 4096)
    ref_kvr = rope(orc_norm(kv_raw, W["kv_a_norm"])[None, :], pos, il)[0]
    assert rel(kvr, ref_kvr) < 1e-5
    # Step 11: the FP8 row that enters the cache
    _, _, _, ref_deq = O.fp8_quant_rows(ref_kvr[None, :])
    check_fp8_emit(kv_fp8.cpu().numpy(), kvr, ref_deq[0], ref_kvr, tol=1e-5, max_flips=2)


def test_attn_qkv_decode_rejects_bad_arguments(gpu, qkv_weights):
    from ds4cuda_amd import Ds4HipError, lib
    x = torch.zeros(4096, device=gpu)
    with pytest.raises(Ds4HipError):
        ops.attn_qkv_decode_f32(x, *(torch.from_numpy(np.ascontiguousarray(qkv_weights[k])).to(gpu)
                                     for k in ("q_a", "q_a_norm", "kv_a", "kv_a_norm", "q_b")),
                                -1, 0, torch.empty(1024, device=gpu), torch.empty(32768, device=gpu),
                                torch.empty(512, device=gpu))
    small = torch.empty(16, dtype=torch.uint8, device=gpu)
    rc = lib().ds4hip_attn_qkv_decode_f32(*([C.c_void_p(x.data_ptr())] * 6), 0, 0,
                                          *([C.c_void_p(x.data_ptr())] * 3), C.c_void_p(small.data_ptr()),
                                          16, None)
    assert rc == -22
