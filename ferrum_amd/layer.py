"""The attention half of one Llama decode layer, GPU-resident.

Llama::forward_one_token (crates/model/src/llama.rs:183-255) runs, per layer, on the
normed hidden row: linear attn_q / attn_k / attn_v (:185-205), Kernels::rope of q and k
at the token's position (:207-216), KvPool::append_layer of k and v (:218), the
attention loop over the sequence's positions (:220-247) and linear attn_output
(:249-255). Here that span is three launches on one stream for a batch of sequences,
each with its own position:

1. fkv_gemm_q8_0_batched: q, k and v from the normed rows, one launch (Q8_0 weights; on
   the matrix cores for batches of 8 sequences or more, the GEMV below that);
2. fkv_rope_append_decode_attention: RoPE of q and k at position ctx_lens[s] - 1, the
   append of k and v through the block tables, decode attention;
3. fkv_gemm_q8_0_batched: attn_output of the attention rows.

Nothing crosses to the host. The activation buffers and the GEMM workspace are allocated
once, for the largest batch the layer was built for; the attention workspace grows when a
call's plan needs more than it holds (the split plan depends on the batch and context, not
monotonically). The buffer it replaces is recorded on every stream that used it, so the
caching allocator hands it out again only after the kernels queued there are done.
"""
from __future__ import annotations

from typing import Optional

from .kvcache import PagedKvPool, default_scale
from .q8 import gemm_q8_0_batched, gemm_q8_0_batched_workspace_bytes, q8_0_row_bytes


class DecodeAttentionLayer:
    """One layer's attention half over `pool` (layer index `layer`).

    wq, wk, wv, wo: device uint8 tensors of Q8_0 rows (ggml order, 34-byte blocks):
    wq [n_heads * head_dim rows x n_embd], wk / wv [n_kv_heads * head_dim x n_embd],
    wo [n_embd x n_heads * head_dim]."""

    def __init__(self, pool: PagedKvPool, layer: int, wq, wk, wv, wo, n_heads: int, n_embd: int,
                 rope_dim: int, theta: float, max_seqs: int, max_ctx_len: int,
                 scale: Optional[float] = None):
        import torch
        cfg = pool.config
        self.pool, self.layer = pool, layer
        self.n_heads, self.n_embd = n_heads, n_embd
        self.hkv, self.d = cfg.n_kv_heads, cfg.head_dim
        self.rope_dim, self.theta = rope_dim, theta
        self.scale = default_scale(self.d) if scale is None else scale
        self.q_rows, self.kv_rows = n_heads * self.d, self.hkv * self.d
        for name, w, rows, cols in (("wq", wq, self.q_rows, n_embd), ("wk", wk, self.kv_rows, n_embd),
                                    ("wv", wv, self.kv_rows, n_embd), ("wo", wo, n_embd, self.q_rows)):
            if w.numel() != rows * q8_0_row_bytes(cols):
                raise ValueError(f"{name} must hold {rows} Q8_0 rows of {cols} columns")
        self.wq, self.wk, self.wv, self.wo = wq, wk, wv, wo
        self.max_seqs, self.max_ctx_len = max_seqs, max_ctx_len
        dev = wq.device
        f32 = torch.float32
        self.q = torch.empty((max_seqs, n_heads, self.d), dtype=f32, device=dev)
        self.k = torch.empty((max_seqs, self.hkv, self.d), dtype=f32, device=dev)
        self.v = torch.empty_like(self.k)
        self.attn = torch.empty_like(self.q)
        need = pool.rope_attention_workspace_bytes(n_heads, max_seqs, max_ctx_len)
        self.ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
        self._ws_streams = {}  # stream handle -> torch stream of each call that used self.ws
        # the quantized activation rows of either GEMM (the launches are stream-ordered)
        # (the size grows with the batch: the largest is the one for max_seqs rows)
        gneed = max(gemm_q8_0_batched_workspace_bytes(n_embd, max_seqs),
                    gemm_q8_0_batched_workspace_bytes(self.q_rows, max_seqs))
        self.gws = torch.empty(max(gneed, 16), dtype=torch.uint8, device=dev)

    def _workspace(self, n: int, max_ctx_len: int, stream):
        import torch
        if stream is None:
            ts = torch.cuda.current_stream(self.ws.device)
        elif isinstance(stream, int):
            ts = torch.cuda.ExternalStream(stream, device=self.ws.device)
        else:
            ts = stream
        need = self.pool.rope_attention_workspace_bytes(self.n_heads, n, max_ctx_len)
        if need > self.ws.numel():
            old = self.ws
            self.ws = torch.empty(need, dtype=torch.uint8, device=old.device)
            # Kernels queued on the streams that used the old buffer may still read or
            # write it: the allocator reuses it only once they have finished.
            for s in self._ws_streams.values():
                old.record_stream(s)
            self._ws_streams = {}
        self._ws_streams[ts.cuda_stream] = ts
        return self.ws

    def forward(self, x, block_tables, ctx_lens, max_ctx_len: int, y, stream=None) -> None:
        """x: device f32 [n_seqs, n_embd], the normed rows (llama.rs:183); y: device f32
        [n_seqs, n_embd] <- attn_output; ctx_lens counts the new token. Also writes each
        sequence's K/V at position ctx_lens[s] - 1 of the layer."""
        n = x.shape[0]
        if n > self.max_seqs or max_ctx_len > self.max_ctx_len:
            raise ValueError("batch or context beyond what the layer was built for")
        if n == 0:
            return
        q, k, v, attn = self.q[:n], self.k[:n], self.v[:n], self.attn[:n]
        gemm_q8_0_batched([self.wq, self.wk, self.wv], [self.q_rows, self.kv_rows, self.kv_rows],
                          self.n_embd, x, n, [q, k, v], workspace=self.gws, stream=stream)
        self.pool.rope_append_decode_attention(self.layer, k, v, q, attn, block_tables, ctx_lens,
                                               max_ctx_len, self.rope_dim, self.theta,
                                               scale=self.scale,
                                               workspace=self._workspace(n, max_ctx_len, stream),
                                               stream=stream)
        gemm_q8_0_batched([self.wo], [self.n_embd], self.q_rows, attn, n, [y],
                          workspace=self.gws, stream=stream)
