"""Tiny causal-LM configurations of the post-head families the head binds (plain, logit scaling, final softcap,
lm_head multiplier) and of the model the reference trains (Qwen3.5: gated-delta-net linear attention layers between
full attention ones, octopus/rl/model_hooks.py:41), with the post-head transform each one implies, and a helper that
packs sequences."""

import numpy as np

# sizes chosen so that every family's attention and mamba shapes divide evenly (mamba: 8 heads x 12 = 2 x hidden)
TINY = dict(vocab_size=112, hidden_size=48, intermediate_size=80, num_hidden_layers=2, num_attention_heads=4,
            num_key_value_heads=2, head_dim=12)
_MAMBA = dict(mamba_n_heads=8, mamba_d_head=12, mamba_d_state=8, mamba_chunk_size=8)
# gated delta net (Qwen3.5's linear attention): 2 key heads and 4 value heads of 8
_GDN = dict(linear_conv_kernel_dim=4, linear_key_head_dim=8, linear_value_head_dim=8, linear_num_key_heads=2,
            linear_num_value_heads=4)
NAMES = ["llama", "granitemoehybrid", "gemma2", "falcon_h1", "qwen3_5"]


def families():
    """[(name, config, post-head transform as (pre, post, tanh))] for the families of NAMES, in that order."""
    from transformers import FalconH1Config, Gemma2Config, GraniteMoeHybridConfig, LlamaConfig
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    return [
        ("llama", LlamaConfig(**TINY), (1.0, 1.0, False)),
        ("granitemoehybrid", GraniteMoeHybridConfig(**TINY, logits_scaling=3.0, layer_types=["mamba", "attention"],
                                                    **_MAMBA), (1 / 3.0, 1.0, False)),
        ("gemma2", Gemma2Config(**TINY, final_logit_softcapping=2.0), (0.5, 2.0, True)),
        ("falcon_h1", FalconH1Config(**TINY, lm_head_multiplier=0.25, mamba_d_ssm=96, **_MAMBA), (0.25, 1.0, False)),
        ("qwen3_5", Qwen3_5TextConfig(**TINY, layer_types=["linear_attention", "full_attention"], **_GDN),
         (1.0, 1.0, False)),
    ]


def packed(seqs):
    """(flat tokens, cumulative offsets [0, len0, len0 + len1, ...]) of a list of token sequences."""
    seqs = [np.asarray(s, dtype=np.int64) for s in seqs]
    offsets = np.zeros(len(seqs) + 1, dtype=np.int64)
    offsets[1:] = np.cumsum([s.size for s in seqs])
    flat = np.concatenate(seqs) if seqs else np.zeros(0, dtype=np.int64)
    return flat, offsets.tolist()
