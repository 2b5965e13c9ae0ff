"""One layer's attention block for a batch of decoding sequences.

This is the batched form of the attention slice of ds4_forward_layer
(Steps 11-16, cuda/forward_layer.cu:915-1210) that cuda/forward_batch.cu:264-284
runs token by token for each sequence. Per step, for every sequence b at
position pos[b] of a compressed layer (ratio 4, with indexer):

  1. attention compressor step (kv / gate projections, APE, state row; on an
     emit step: softmax pool, RMSNorm, tail RoPE at pos + 1 - 4, FP8 round
     trip) and indexer compressor step (the same at width 128, no FP8);
  2. the token's KV row -> FP8 into its sliding-window slot (pos % 128), the
     emitted compressed row -> FP8 into the next compressed row, the emitted
     indexer key -> the sequence's key rows;
  3. indexer top-k over the sequence's compressed rows (fp32 keys);
  4. decode attention over the 128 window rows plus the selected compressed
     rows (paged FP8 cache, sink per head);
  5. inverse tail RoPE of the 64 heads' outputs at pos;
  6. the output projection 64 x 512 -> out_dim (bf16 weights).

Cache layout: sequence b owns logical rows [0, cap_comp) (compressed rows, in
emit order) and [cap_comp, cap_comp + 128) (the window ring, slot pos % 128);
logical row l lives at physical row page_table[b][l // page_rows] *
page_rows + l % page_rows. Rows of sequences that do not emit this step go to
one spare ("trash") row, so the step's launches do not depend on which
sequences emit. The window must be full (pos >= 127 for every sequence), as
in the configurations this block serves.

Every kernel is a libds4hip.so entry point; torch provides device memory and
the stream only.
"""
from __future__ import annotations

import numpy as np
import torch

from . import ops
from ._lib import Ds4HipError, call
from .ops import _ptr, _stream

N_HEAD, HEAD_DIM, N_ROT, IDX_DIM, SWA, RATIO = 64, 512, 64, 128, 128, 4


class BatchedAttentionBlock:
    """weights: dict of device tensors
         w_kv, w_gate [2*512, in_dim] fp32;  ape [4, 1024] f16 bits (int16);
         wn [512] fp32;  wi_kv, wi_gate [2*128, in_dim] fp32;  ape_i [4, 256];
         wn_i [128];  w_out [out_dim, 64*512] bf16.
    max_pos: largest position a step may decode (sizes the caches)."""

    def __init__(self, weights, n_seq, max_pos, in_dim=4096, out_dim=4096, page_rows=256,
                 top_k=2048, il=2, device="cuda", page_seed=6, fused=True):
        if n_seq > 16:
            raise Ds4HipError("at most 16 sequences per batched block", -22)
        self.w = weights
        self.B, self.in_dim, self.out_dim = n_seq, in_dim, out_dim
        self.page_rows, self.top_k, self.il, self.dev = page_rows, top_k, il, device
        self.cap_comp = (max_pos + 1) // RATIO + 1
        lrows = self.cap_comp + SWA
        self.pages_per = (lrows + page_rows - 1) // page_rows
        perm = np.random.default_rng(page_seed).permutation(n_seq * self.pages_per)
        self.pt_host = perm.reshape(n_seq, self.pages_per).astype(np.int32)
        self.page_table = torch.from_numpy(self.pt_host).to(device)
        self.trash = n_seq * self.pages_per * page_rows
        self.cache = ops.Fp8KVCache.empty(self.trash + 1, device=device)
        self.key_cap = self.cap_comp
        self.key_trash = n_seq * self.key_cap
        self.keys = torch.zeros((self.key_trash + 1, IDX_DIM), device=device)
        self.key_row0 = (np.arange(n_seq) * self.key_cap).astype(np.int64)
        B = n_seq
        self.st_kv = torch.zeros((B, 8, 1024), device=device)
        self.st_sc = torch.full((B, 8, 1024), float("-inf"), device=device)
        self.sti_kv = torch.zeros((B, 8, 256), device=device)
        self.sti_sc = torch.full((B, 8, 256), float("-inf"), device=device)
        self.emit = torch.zeros((B, HEAD_DIM), device=device)
        self.emit_i = torch.zeros((B, IDX_DIM), device=device)
        self.scratch = ops.compressor_batch_scratch(B, in_dim, HEAD_DIM, RATIO, device)
        self.scratch_i = ops.compressor_batch_scratch(B, in_dim, IDX_DIM, RATIO, device)
        # fused: both compressors in three launches (ds4hip_compressor_pair_step_batch_w32)
        # instead of six, the three row pushes in one (ds4hip_batch_rows_push_f32), and
        # the inverse RoPE in the decode's merge; the same results
        self.fused = fused
        self.scratch_pair = ops.compressor_pair_scratch(B, in_dim, HEAD_DIM, IDX_DIM, RATIO, device)
        self.mm_ws = ops.mul_mm_workspace(out_dim, N_HEAD * HEAD_DIM, B, device)
        self.scores = torch.empty(self.key_trash + 1, device=device)
        self.out = torch.empty((B, N_HEAD, HEAD_DIM), device=device)
        self.y = torch.empty((B, out_dim), device=device)
        self._plans = {}

    # ---- host-side layout ------------------------------------------------------
    def phys(self, b, lrow):
        return int(self.pt_host[b][lrow // self.page_rows]) * self.page_rows + lrow % self.page_rows

    def window_lrow(self, pos):
        return self.cap_comp + pos % SWA

    def load_history(self, b, comp_rows, window_rows, window_pos, keys, stream=None):
        """Sequence b's state before a step: comp_rows [n, 512] fp32 (the
        emitted compressed rows, in order), window_rows [m, 512] fp32 for token
        positions window_pos [m], keys [n, 128] fp32 (indexer keys)."""
        n = comp_rows.shape[0]
        if n > self.cap_comp or keys.shape[0] != n:
            raise Ds4HipError("history larger than the block's capacity", -22)
        dst = [self.phys(b, l) for l in range(n)]
        dst += [self.phys(b, self.window_lrow(int(p))) for p in window_pos]
        rows = torch.cat([comp_rows, window_rows]).contiguous()
        self.cache.append(rows, dst_rows=torch.tensor(dst, dtype=torch.int64, device=self.dev),
                          stream=stream)
        if n:
            dk = torch.arange(self.key_row0[b], self.key_row0[b] + n, dtype=torch.int64,
                              device=self.dev)
            call("ds4hip_rows_scatter_f32", _ptr(keys.contiguous()), n, IDX_DIM,
                 _ptr(self.keys), _ptr(dk), _stream(stream))

    def plan(self, pos):
        """Host-decided arguments of a step at positions pos (cached per pos)."""
        key = tuple(int(p) for p in pos)
        if key in self._plans:
            return self._plans[key]
        if min(key) < SWA - 1:
            raise Ds4HipError("the batched block needs a full window (pos >= 127)", -22)
        n_before = [p // RATIO for p in key]
        emits = [(p + 1) % RATIO == 0 for p in key]
        n_after = [n + int(e) for n, e in zip(n_before, emits)]
        if max(n_after) > self.cap_comp:
            raise Ds4HipError("position beyond the block's capacity", -22)
        d = self.dev
        dst_raw = [self.phys(b, self.window_lrow(p)) for b, p in enumerate(key)]
        dst_emit = [self.phys(b, n_before[b]) if emits[b] else self.trash for b in range(self.B)]
        dst_key = [int(self.key_row0[b]) + n_before[b] if emits[b] else self.key_trash
                   for b in range(self.B)]
        win = np.array([[self.window_lrow(p - k) for k in range(SWA)] for p in key], np.int32)
        plan = {
            "pos_host": np.array(key, np.int32),
            "pos_dev": torch.tensor(key, dtype=torch.int32, device=d),
            "dst_raw": torch.tensor(dst_raw, dtype=torch.int64, device=d),
            "dst_emit": torch.tensor(dst_emit, dtype=torch.int64, device=d),
            "dst_key": torch.tensor(dst_key, dtype=torch.int64, device=d),
            # row lists: the window rows (constant per position), then the
            # selected compressed rows the indexer writes each step
            "rowlist": torch.cat([torch.from_numpy(win),
                                  torch.zeros((self.B, self.top_k), dtype=torch.int32)],
                                 dim=1).to(d).contiguous(),
            "n_comp": n_after,
            "counts": [SWA + min(n, self.top_k) for n in n_after],
            "emits": emits,
        }
        plan["ws"] = torch.empty(ops.decode_fp8_workspace_bytes(plan["counts"]),
                                 dtype=torch.uint8, device=d)
        self._plans[key] = plan
        return plan

    # ---- one step ----------------------------------------------------------------
    def step(self, pos, x, kv_cur, q, q_idx, w_idx, sinks, stream=None):
        """x [B, in_dim] fp32 (the normed layer input), kv_cur [B, 512] fp32
        (the token's KV row after its tail RoPE), q [B, 64, 512] bf16, q_idx
        [B, 64, 128] fp32, w_idx [B, 64] fp32 (indexer head weights, already
        scaled), sinks [B, 64] fp32. Returns y [B, out_dim] fp32."""
        P = self.plan(pos)
        w, B = self.w, self.B
        if self.fused:
            ops.compressor_pair_step_batch_w32(
                x, self.in_dim, RATIO, P["pos_host"], P["pos_dev"], self.il,
                dict(w_kv=w["w_kv"], w_gate=w["w_gate"], w_ape=w["ape"], w_norm=w["wn"], head_dim_out=HEAD_DIM,
                     state_kv=self.st_kv, state_score=self.st_sc, state_stride=8 * 1024, emit_out=self.emit),
                dict(w_kv=w["wi_kv"], w_gate=w["wi_gate"], w_ape=w["ape_i"], w_norm=w["wn_i"],
                     head_dim_out=IDX_DIM, state_kv=self.sti_kv, state_score=self.sti_sc, state_stride=8 * 256,
                     emit_out=self.emit_i),
                self.scratch_pair, stream=stream)
        else:
            ops.compressor_decode_step_batch_w32(True, x, w["w_kv"], w["w_gate"], w["ape"], w["wn"],
                                                 self.in_dim, HEAD_DIM, RATIO, P["pos_host"],
                                                 P["pos_dev"], self.il, self.st_kv, self.st_sc,
                                                 8 * 1024, self.emit, self.scratch, stream=stream)
            ops.compressor_decode_step_batch_w32(False, x, w["wi_kv"], w["wi_gate"], w["ape_i"],
                                                 w["wn_i"], self.in_dim, IDX_DIM, RATIO, P["pos_host"],
                                                 P["pos_dev"], self.il, self.sti_kv, self.sti_sc,
                                                 8 * 256, self.emit_i, self.scratch_i, stream=stream)
        if self.fused:   # the three row pushes in one launch
            ops.batch_rows_push_f32(self.cache, ((kv_cur, P["dst_raw"]), (self.emit, P["dst_emit"])), self.emit_i,
                                    self.keys, P["dst_key"], stream=stream)
        else:
            self.cache.append(kv_cur, dst_rows=P["dst_raw"], stream=stream)
            self.cache.append(self.emit, dst_rows=P["dst_emit"], stream=stream)
            call("ds4hip_rows_scatter_f32", _ptr(self.emit_i), B, IDX_DIM, _ptr(self.keys),
                 _ptr(P["dst_key"]), _stream(stream))
        self.rowlist = P["rowlist"]
        ops.indexer_topk_positions_batch(q_idx, w_idx, self.keys, self.key_row0, P["n_comp"],
                                         self.top_k, 0, self.scores, self.rowlist,
                                         pos_offset=SWA, stream=stream)
        if self.fused:   # the merge writes the inverse-RoPE'd rows
            ops.flash_attn_decode_fp8(q, sinks, self.out, self.cache, P["counts"],
                                      row_idx=self.rowlist, page_table=self.page_table,
                                      page_rows=self.page_rows, workspace=P["ws"],
                                      rope_out=(P["pos_dev"], self.il), stream=stream)
        else:
            ops.flash_attn_decode_fp8(q, sinks, self.out, self.cache, P["counts"],
                                      row_idx=self.rowlist, page_table=self.page_table,
                                      page_rows=self.page_rows, workspace=P["ws"], stream=stream)
            ops.tail_rope_yarn_batch_f32(self.out, self.out, B, N_HEAD, HEAD_DIM, N_ROT,
                                         P["pos_dev"], self.il, inverse=True, stream=stream)
        ops.mul_mm_bf16_f32(w["w_out"], self.out, self.y, self.out_dim, N_HEAD * HEAD_DIM, B,
                            workspace=self.mm_ws, stream=stream)
        return self.y

    def capture(self, pos, x, kv_cur, q, q_idx, w_idx, sinks):
        """Records one step() with these arguments into a HIP graph
        (torch.cuda.CUDAGraph) and returns it; graph.replay() runs the step
        again on the same buffers with one launch of the graph instead of the
        step's 13 kernel launches. Nothing in step() allocates, synchronizes
        the host or writes memory with hipMemsetAsync, so the graph holds
        kernel nodes only; the host-side plan for pos is built before the
        capture. Each replay advances the block's state as an eager step()
        would (compressor states, appended rows)."""
        self.plan(pos)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(g, stream=side):
                self.step(pos, x, kv_cur, q, q_idx, w_idx, sinks, stream=side)
        torch.cuda.current_stream().wait_stream(side)
        return g
