"""The BASELINE workload configurations, as ut_model_config dictionaries.

C1: tiny DeepSeek-V3-style model (the reference's OracleSpec at config-1
dimensions); C4: truncated-depth DeepSeek-V3 at full width.  C2 (isolated
expert block) and C3 (MLA decode attention) are kernel shapes.
"""

C1 = dict(vocab_size=1024, hidden_size=256, intermediate_size=512, moe_intermediate_size=128,
          num_hidden_layers=2, first_k_dense_replace=1, num_attention_heads=4,
          n_routed_experts=8, num_experts_per_tok=2, n_shared_experts=1, n_group=4, topk_group=2,
          norm_topk_prob=1, routed_scaling_factor=2.5, q_lora_rank=96, kv_lora_rank=64,
          qk_nope_head_dim=32, qk_rope_head_dim=16, v_head_dim=32, rms_norm_eps=1e-6,
          rope_theta=10000.0, mtp=1, max_position_embeddings=4096)

# DeepSeek-V3 widths (config.json of deepseek-ai/DeepSeek-V3) at 4 layers.
C4 = dict(vocab_size=129280, hidden_size=7168, intermediate_size=18432,
          moe_intermediate_size=2048, num_hidden_layers=4, first_k_dense_replace=1,
          num_attention_heads=128, n_routed_experts=256, num_experts_per_tok=8,
          n_shared_experts=1, n_group=8, topk_group=4, norm_topk_prob=1,
          routed_scaling_factor=2.5, q_lora_rank=1536, kv_lora_rank=512, qk_nope_head_dim=128,
          qk_rope_head_dim=64, v_head_dim=128, rms_norm_eps=1e-6, rope_theta=10000.0, mtp=1,
          max_position_embeddings=1024)

# C5: DeepSeek-V3 671B's shape at full depth (61 layers, the first 3 dense),
# context for a 2048-token prompt plus 256 new tokens.  Its routed experts
# (59 MoE layers with the MTP module x 256 x 22 MB = 333 GB int4) exceed HBM
# and run behind the expert store's HBM tier.
C5 = dict(C4, num_hidden_layers=61, first_k_dense_replace=3, max_position_embeddings=2560)

# C2: one routed-expert block at DeepSeek-V3 expert shape.
C2 = dict(hidden=7168, inter=2048, n_experts=256, top_k=8, n_group=8, topk_group=4,
          norm_topk_prob=1, routed_scaling_factor=2.5)

# Algorithmic bytes of one expert (gate + up [2048, 7168] + down [7168, 2048],
# payload + per-row f32 scales).
def expert_bytes(hidden: int, inter: int, fmt_bits: int) -> int:
    per = lambda o, i: o * ((i * fmt_bits + 7) // 8) + o * 4
    return 2 * per(inter, hidden) + per(hidden, inter)


def gate_up_bytes(hidden: int, inter: int, fmt_bits: int) -> int:
    return 2 * (inter * ((hidden * fmt_bits + 7) // 8) + inter * 4)
