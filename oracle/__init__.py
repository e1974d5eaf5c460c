"""CPU oracle of tessery's prefill-attention path (float64 NumPy).

TEST INFRASTRUCTURE ONLY. It is imported by tests/, by __graft_entry__.smoke() and by bench.py's
CPU-baseline leg, and only as the reference results or the timed CPU baseline. The product path
(tessery_amd) never imports, calls or falls back to it.

Modules and what pins each one (the tests under tests/test_oracle_*.py run these checks):
  attention   per-(batch, head) softmax attention with tessery's mask / padding / GQA semantics.
              Pinned by torch.nn.functional.scaled_dot_product_attention (float64, enable_gqa,
              explicit tril & key-padding masks), the closed-form known answers of tessery's
              extreme-logit test (test_kernels.py:213-253) and a scalar online-softmax loop.
  norm_rope   per-head RMSNorm and split-half RoPE. Pinned by torch.nn.functional.rms_norm,
              transformers' Qwen3RMSNorm / apply_rotary_pos_emb, a complex-number rotation and
              rotation invariants.
  quant4      uint4 group-64 packing, dequantization and projection, silu_gate and the fused
              gate/up projection. Pinned by tessery's known-answer tests (test_kernels.py:55-81,
              286-294, 759-776, 842-857), a scalar restatement of the kernel indexing
              (kernels.metal:11-19), torch's silu and transformers' Qwen3MLP.
  qwen_block  compositions of the Qwen3 layer: QKV projection -> q/k norm + RoPE -> attention
              (qwen3.py:194-245), pinned through the modules above, and the layer tail o_proj ->
              residual -> RMSNorm -> gate/up + SiLU -> down -> residual (qwen3.py:246-280), pinned
              against torch's rms_norm and transformers' Qwen3MLP.
  bert_block  the BERT (BGE) encoder layer (bert.py:186-230): fp32 projections with bias, GELU,
              LayerNorm and bidirectional attention. Pinned against torch's gelu / layer_norm,
              math.erf and transformers' BertLayer in float64 with a key-padding mask.
  models      whole forwards: embedding4 / embedding_position gathers (kernels.metal:21-30,
              351-360), pool_project (kernels.metal:339-349), the Qwen3 forward (qwen3.py:112-296)
              and the BERT forward (bert.py:103-251). Pinned by the scalar weight4 indexing, the
              pooling definition, and transformers' Qwen3Model and BertModel in float64 on the same
              weights (1e-10), with planted mistakes (wrong pooled token, a dropped layer).
No function here is "parity unpinned".
"""
