"""The scalar-operand exact scorer (score_sgpr_kernel, selected with
DS4HIP_INDEXER_SGPR_SCORES=1 at launch) against the default LDS scorer and
the oracle: bit-identical scores and positions for f32, f16 and bf16 keys,
a ragged key count and the cfg 3 size with planted ties."""
import ctypes as C
import os

import numpy as np
import pytest
import torch

import oracle as O
from oracle import P
from ds4cuda_amd import ops, synth
from unverified import unverified

pytestmark = pytest.mark.gpu


@unverified("the scalar-operand scorer has not run on the GPU yet")
@pytest.mark.parametrize("kind,n_comp", [(0, 1000), (1, 4097), (2, 131072)])
def test_sgpr_scorer_bit_identical(gpu, kind, n_comp):
    n_head, hd, top_k, recent = 64, 128, 512, 128
    q = synth.normal(91, 1, n_head * hd)
    w = synth.normal(91, 2, n_head) / np.float32(np.sqrt(hd * n_head))
    kf = synth.normal(91, 3, n_comp * hd).reshape(n_comp, hd)
    kf[100:140] = kf[7]
    if kind == 0:
        keys, kt = kf, torch.from_numpy(kf).to(gpu)
    elif kind == 1:
        keys = kf.astype(np.float16)
        kt = torch.from_numpy(keys).to(gpu)
    else:
        keys = synth.to_bf16_bits(kf)
        kt = torch.from_numpy(keys.view(np.int16)).to(gpu).view(torch.bfloat16)
    ref_s = np.zeros(n_comp, np.float32)
    O.lib().orc_indexer_scores(P(q), P(w), P(np.ascontiguousarray(keys)), C.c_int(kind), C.c_int(n_comp),
                               C.c_int(n_head), C.c_int(hd), P(ref_s))
    ref_p = np.zeros(top_k, np.int32)
    O.lib().orc_topk_positions(P(ref_s), C.c_int(n_comp), C.c_int(top_k), C.c_int(recent), P(ref_p))
    qt, wt = torch.from_numpy(q).to(gpu), torch.from_numpy(w).to(gpu)
    got = {}
    prev = os.environ.get("DS4HIP_INDEXER_SGPR_SCORES")
    try:
        for mode in ("0", "1"):
            os.environ["DS4HIP_INDEXER_SGPR_SCORES"] = mode
            pos, _, scores = ops.indexer_topk_positions(qt, wt, kt.view(n_comp, hd), top_k, recent)
            torch.cuda.synchronize()
            got[mode] = (pos.cpu().numpy().copy(), scores.cpu().numpy().copy())
    finally:
        if prev is None:
            os.environ.pop("DS4HIP_INDEXER_SGPR_SCORES", None)
        else:
            os.environ["DS4HIP_INDEXER_SGPR_SCORES"] = prev
    for mode in ("0", "1"):
        pos, sc = got[mode]
        assert np.array_equal(sc.view(np.uint32), ref_s.view(np.uint32)), mode
        assert np.array_equal(np.sort(pos[:top_k]), ref_p), mode
