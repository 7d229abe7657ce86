"""Host-side logic of the product on the CPU: the prefix-tree pairs against the oracle's trie, the reference's
own CPU head tests (tests/test_lm_head.py of the reference) through octopus_amd.rl.lm_head, the post-head
chain parsing the fused epilogue relies on, and the seq-tile entry points."""

import numpy as np
import pytest
import torch

from octopus_amd.rl import lm_head, prefix_tree, seq_tiles
from octopus_amd.rl.lm_head import _fused_post, bind_head
from octopus_amd.rl.prefix_tree import TreeMeta, build_tree, tree_head_output
from oracle import pairs as opairs

SMALL = dict(vocab_size=96, hidden_size=32, intermediate_size=64, num_hidden_layers=2, num_attention_heads=2,
             num_key_value_heads=1, head_dim=16)


def _flat(seqs):
    return np.concatenate(seqs), [0, *np.cumsum([len(s) for s in seqs]).tolist()]


def _random_forest(rng, n_seq):
    """Sequences sharing prefixes at random depths, duplicates and empties included."""
    base = [rng.integers(0, 6, rng.integers(1, 30)) for _ in range(3)]
    seqs = []
    for _ in range(n_seq):
        b = base[rng.integers(0, 3)]
        cut = int(rng.integers(0, len(b) + 1))
        seqs.append(np.concatenate([b[:cut], rng.integers(0, 6, rng.integers(0, 8))]))
    return seqs


@pytest.mark.parametrize("seed", range(12))
def test_build_tree_matches_the_trie_oracle(seed):
    rng = np.random.default_rng(seed)
    seqs = _random_forest(rng, int(rng.integers(1, 9)))
    flat, cu = _flat(seqs)
    if len(flat) == 0:
        return
    scored = None if seed % 3 == 0 else rng.random(len(flat)) < 0.5
    tree = build_tree(flat, cu, scored=scored)
    tokens, f2t, posid = opairs.tree_positions(flat, cu)
    assert np.array_equal(tree.tokens, tokens) and np.array_equal(tree.position_ids, posid)
    assert np.array_equal(tree.flat_to_tree, f2t)
    pos, lab, fp = opairs.pairs(flat, cu, scored)
    assert np.array_equal(tree.pair_pos, pos) and np.array_equal(tree.pair_label, lab)
    assert np.array_equal(tree.flat_pair, fp)
    for node in tree.nodes:  # pre-order ranges tile the tree; a node's path ends with its own tokens
        assert (node.path[-(node.end - node.start):] == np.arange(node.start, node.end)).all()


def test_build_tree_reference_cases():
    flat, cu = _flat([np.array([1, 2, 3, 4]), np.array([1, 2, 9])])
    tree = build_tree(flat, cu)
    assert tree.tokens.tolist() == [1, 2, 3, 4, 9]
    flat, cu = _flat([np.array([5, (1 << 21) + 3, 7]), np.array([5, (1 << 21) + 3, (1 << 20) + 9])])
    tree = build_tree(flat, cu)
    for p in (0, 1, 3, 4):
        row = tree.flat_pair[p]
        assert tree.tokens[tree.pair_pos[row]] == flat[p] and tree.pair_label[row] == flat[p + 1]
    with pytest.raises(NotImplementedError):
        build_tree(flat, cu, mounts={1: [(1, 0, 0, 2)]})


def test_tree_head_output_expands_pairs_to_flat_positions():
    """Reference tests/test_prefix_tree.py:165-176 through the product's tree_head_output."""
    flat, cu = _flat([np.array([1, 2, 3, 4]), np.array([1, 2, 9])])
    meta = TreeMeta(build_tree(flat, cu), "cpu")
    hidden = torch.arange(5, dtype=torch.float32)[None, :, None]

    def head(rows, labels):
        return torch.stack([rows[:, 0] * 10 + labels, labels.float()], -1)

    out = tree_head_output(head, hidden, meta)[0]
    assert out[1, 1] == 3 and out[5, 1] == 9 and out[1, 0] == 1 * 10 + 3 and out[5, 0] == 1 * 10 + 9
    assert (out[[3, 6]] == 0).all()


def _families():
    from transformers import FalconH1Config, Gemma2Config, GraniteMoeHybridConfig, LlamaConfig
    return [
        LlamaConfig(**SMALL),
        GraniteMoeHybridConfig(**SMALL, logits_scaling=3.0, layer_types=["mamba", "attention"], mamba_n_heads=4,
                               mamba_d_head=16, mamba_d_state=8, mamba_chunk_size=8),
        Gemma2Config(**SMALL, final_logit_softcapping=2.0),
        FalconH1Config(**SMALL, lm_head_multiplier=0.25, mamba_n_heads=4, mamba_d_head=16, mamba_d_ssm=64,
                       mamba_d_state=8, mamba_chunk_size=8),
    ]


EXPECTED_POST = [dict(pre=1.0, post=1.0, tanh=False), dict(pre=1 / 3.0, post=1.0, tanh=False),
                 dict(pre=0.5, post=2.0, tanh=True), dict(pre=0.25, post=1.0, tanh=False)]


@pytest.mark.parametrize("k", range(4), ids=["llama", "granitemoehybrid", "gemma2", "falcon_h1"])
def test_chunked_head_matches_the_models_own_logits(k):
    """Reference tests/test_lm_head.py:11-34 (CPU, fp32, atol 1e-5), and the fused epilogue's reading of the
    recorded post-head chain."""
    from transformers import AutoModelForCausalLM
    config = _families()[k]
    torch.manual_seed(0)
    model = AutoModelForCausalLM.from_config(config, attn_implementation="eager").eval()
    ids = torch.randint(0, config.vocab_size, (1, 12))
    labels = torch.roll(ids, -1, -1).reshape(-1)
    with torch.no_grad():
        own = model(input_ids=ids).logits[0].float()
    for temperature in (1.0, 0.7):
        head = bind_head(model, temperature)
        head.octopus_labels, head.octopus_tree = labels, None
        with torch.no_grad():
            out = model(input_ids=ids).logits[0]
        logp = torch.log_softmax(own / temperature, -1)
        assert torch.allclose(out[:, 0], logp.gather(-1, labels[:, None])[:, 0], atol=1e-5)
        assert torch.allclose(out[:, 1], -(logp.exp() * logp).sum(-1), atol=1e-5)
    assert bool(head.octopus_post) == (config.model_type != "llama")
    post = _fused_post(head.octopus_post)
    exp = EXPECTED_POST[k]
    assert abs(post.pre - exp["pre"]) < 1e-12 and abs(post.post - exp["post"]) < 1e-12 and post.tanh == exp["tanh"]


@pytest.mark.parametrize("tail", [
    lambda m, logits: (logits.__setitem__((..., 0), 0.0), logits)[1],  # masked in place
    lambda m, logits: (logits * 2, logits / 3)[1],  # an op on an earlier result
    lambda m, logits: m.extra(logits),  # a submodule after the head
], ids=["setitem", "fork", "submodule"])
def test_unreproducible_post_head_logits_fail_loudly(tail):
    """Reference tests/test_lm_head.py:37-55."""
    from transformers import LlamaConfig
    from transformers.modeling_outputs import CausalLMOutput
    from transformers.models.llama.modeling_llama import LlamaForCausalLM

    class Model(LlamaForCausalLM):
        def __init__(self, config):
            super().__init__(config)
            self.extra = torch.nn.Linear(config.vocab_size, config.vocab_size)

        def forward(self, input_ids=None, **kwargs):
            return CausalLMOutput(logits=tail(self, self.lm_head(self.model(input_ids=input_ids).last_hidden_state)))

    with pytest.raises(NotImplementedError):
        bind_head(Model(LlamaConfig(**SMALL)), 1.0)


def test_flat_head_runs_only_the_scored_positions():
    """Reference tests/test_lm_head.py:58-75 (fp64, exact)."""
    from transformers import AutoModelForCausalLM, LlamaConfig
    torch.manual_seed(0)
    model = AutoModelForCausalLM.from_config(LlamaConfig(**SMALL), attn_implementation="eager").double()
    ids = torch.randint(0, SMALL["vocab_size"], (1, 12))
    head = bind_head(model, 0.7)
    head.octopus_labels, head.octopus_tree = torch.roll(ids, -1, -1).reshape(-1), None
    scored = torch.rand(12) < 0.4
    w = torch.randn(1, 12, 2, dtype=torch.float64) * scored[None, :, None]
    outs, grads = [], []
    for head.octopus_scored in (None, scored):
        model.zero_grad(set_to_none=True)
        out = model(input_ids=ids).logits
        (out * w).sum().backward()
        outs.append(out.detach()[0])
        grads.append([p.grad for p in model.parameters()])
    assert torch.equal(outs[1][scored], outs[0][scored]) and (outs[1][~scored] == 0).all()
    assert all(torch.equal(a, b) for a, b in zip(*grads))


def test_fused_post_rejects_chains_without_an_epilogue():
    with pytest.raises(NotImplementedError):
        _fused_post([(torch.Tensor.__add__, (lm_head._LOGITS, 1.0), {})])
    with pytest.raises(NotImplementedError):
        _fused_post([(torch.Tensor.__mul__, (lm_head._LOGITS, -2.0), {})])
    p = _fused_post([(torch.Tensor.__truediv__, (lm_head._LOGITS, 4.0), {}), (torch.tanh, (lm_head._LOGITS,), {}),
                     (torch.Tensor.__mul__, (lm_head._LOGITS, 4.0), {})])
    assert (p.pre, p.post, p.tanh) == (0.25, 4.0, True)


def test_head_columns_is_a_monkeypatchable_global_with_an_eager_twin(monkeypatch):
    """The reference's tests swap lm_head._head_columns (tests/test_actor_chunk_major.py:33) and read
    `_torchdynamo_orig_callable` (tests/test_seq_tiles.py:157)."""
    calls = []
    real = lm_head._head_columns
    assert real._torchdynamo_orig_callable is not real
    monkeypatch.setattr(lm_head, "_head_columns", lambda lg, T, y: calls.append(1) or real(lg, T, y))
    w = torch.randn(7, 5)
    lm_head._head_chunk(w, 1.0, [], torch.randn(3, 5), torch.tensor([0, 1, 6]))
    assert calls


def test_tiled_and_no_inner():
    x = torch.randn(1, 10, 3, requires_grad=True)
    old = seq_tiles.TILE
    try:
        seq_tiles.TILE = 4
        y = seq_tiles.tiled(lambda a: a * 2, x)
        assert torch.equal(y, x * 2)
        y.sum().backward()
        assert torch.equal(x.grad, torch.full_like(x, 2.0))
        with seq_tiles.no_inner():
            assert seq_tiles._INNER is False
        assert seq_tiles._INNER is True
        a, b = seq_tiles.tiled(lambda p, q: (p + 1, q), x, None if False else x)
        assert a.shape == x.shape and torch.equal(b, x)
    finally:
        seq_tiles.TILE = old


def test_prefix_tree_module_exports():
    assert callable(prefix_tree.build_tree) and callable(prefix_tree.tree_head_output)


def test_gather_flag_asks_for_the_row_copy_only_past_2_gib_through_idx():
    """The torch op requests OCTO_WS_GATHER exactly when rows are read through idx from a matrix whose rows x row
    stride x element bytes reach 2^31 - 1, the C ABI's own test (meta tensors: shapes and strides, no memory)."""
    from octopus_amd import _lib
    from octopus_amd.head_op import _gather_flag
    idx = torch.zeros(4, dtype=torch.int64)
    small = torch.empty_strided((262_143, 4096), (4096, 1), dtype=torch.bfloat16, device="meta")  # 2^31 - 2^13 B
    big = torch.empty_strided((262_144, 4096), (4096, 1), dtype=torch.bfloat16, device="meta")    # 2^31 B
    wide = torch.empty_strided((131_072, 4096), (8192, 1), dtype=torch.bfloat16, device="meta")   # strided: 2^31 B
    assert _gather_flag(small, idx) == 0
    assert _gather_flag(big, idx) == _lib.WS_GATHER
    assert _gather_flag(wide, idx) == _lib.WS_GATHER
    assert _gather_flag(big, None) == 0  # without idx each tile's rows are addressed from their own base
