"""Tiny causal-LM configurations of the four post-head families the head binds (plain, logit scaling, final softcap,
lm_head multiplier), with the post-head transform each one implies, and a helper that packs sequences."""

import numpy as np

# sizes chosen so that every family's attention and mamba shapes divide evenly (mamba: 8 heads x 12 = 2 x hidden)
TINY = dict(vocab_size=112, hidden_size=48, intermediate_size=80, num_hidden_layers=2, num_attention_heads=4,
            num_key_value_heads=2, head_dim=12)
_MAMBA = dict(mamba_n_heads=8, mamba_d_head=12, mamba_d_state=8, mamba_chunk_size=8)


def families():
    """[(name, config, post-head transform as (pre, post, tanh))] for the four families."""
    from transformers import FalconH1Config, Gemma2Config, GraniteMoeHybridConfig, LlamaConfig
    return [
        ("llama", LlamaConfig(**TINY), (1.0, 1.0, False)),
        ("granitemoehybrid", GraniteMoeHybridConfig(**TINY, logits_scaling=3.0, layer_types=["mamba", "attention"],
                                                    **_MAMBA), (1 / 3.0, 1.0, False)),
        ("gemma2", Gemma2Config(**TINY, final_logit_softcapping=2.0), (0.5, 2.0, True)),
        ("falcon_h1", FalconH1Config(**TINY, lm_head_multiplier=0.25, mamba_d_ssm=96, **_MAMBA), (0.25, 1.0, False)),
    ]


def packed(seqs):
    """(flat tokens, cumulative offsets [0, len0, len0 + len1, ...]) of a list of token sequences."""
    seqs = [np.asarray(s, dtype=np.int64) for s in seqs]
    offsets = np.zeros(len(seqs) + 1, dtype=np.int64)
    offsets[1:] = np.cumsum([s.size for s in seqs])
    flat = np.concatenate(seqs) if seqs else np.zeros(0, dtype=np.int64)
    return flat, offsets.tolist()
