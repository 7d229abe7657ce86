"""Host-side logic of the product on the CPU: the prefix-tree pairs against the oracle's trie, the properties the
reference's CPU head tests check (tests/test_lm_head.py:11-75, tests/test_prefix_tree.py:165-176 of the reference)
restated through octopus_amd.rl.lm_head, the post-head chain parsing the fused epilogue relies on, and the seq-tile
entry points."""

import numpy as np
import pytest
import torch

from octopus_amd.rl import lm_head, prefix_tree, seq_tiles
from octopus_amd.rl.lm_head import _fused_post, bind_head
from octopus_amd.rl.prefix_tree import TreeMeta, build_tree, tree_head_output
from oracle import pairs as opairs
from tests.tiny_models import NAMES, TINY, families, packed


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
    flat, cu = packed(seqs)
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
    for node in tree.nodes:  # the last (end - start) entries of a node's path are its own tree range, in order
        own = np.arange(node.start, node.end)
        assert np.array_equal(node.path[len(node.path) - own.size:], own)


def test_build_tree_reference_cases():
    flat, cu = packed([[1, 2, 3, 4], [1, 2, 9]])
    assert build_tree(flat, cu).tokens.tolist() == [1, 2, 3, 4, 9]
    big = (1 << 21) + 3  # token ids past 2^20
    flat, cu = packed([[5, big, 7], [5, big, (1 << 20) + 9]])
    tree = build_tree(flat, cu)
    for p in (0, 1, 3, 4):  # each position that asks: its pair's hidden row holds its own token, the label the next
        pos, lab = tree.pair_pos[tree.flat_pair[p]], tree.pair_label[tree.flat_pair[p]]
        assert (tree.tokens[pos], lab) == (flat[p], flat[p + 1])
    with pytest.raises(NotImplementedError):
        build_tree(flat, cu, mounts={1: [(1, 0, 0, 2)]})


def _next_token_expectation(flat, cu, scored, f2t, fn):
    """[T_flat, C] by definition: position p that asks (scored, and not its sequence's last) gets fn(tree position
    of p, flat[p + 1]); every other position a zero row."""
    rows = []
    ends = set(int(e) - 1 for e in cu[1:])
    for p in range(len(flat)):
        asks = p not in ends and (scored is None or bool(scored[p]))
        rows.append(fn(int(f2t[p]), int(flat[p + 1])) if asks else [0.0, 0.0])
    return torch.tensor(rows, dtype=torch.float64)


@pytest.mark.parametrize("case", [0, 1, 2, 3])
def test_tree_head_output_gives_each_position_its_own_next_token(case):
    """The expansion of reference tests/test_prefix_tree.py:165-176, stated as a property: through tree_head_output,
    every flat position that asks gets the head's value at (its own tree row, its own next flat token), shared
    prefixes with different continuations included, and every other position exactly zero. Cases: the reference's
    hand-built forests and a random deduplicated one (tests/golden/prefix_pairs.json)."""
    import json
    import os
    fx = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "prefix_pairs.json")))[case]
    flat, cu = np.array(fx["flat"], dtype=np.int64), np.array(fx["cu"], dtype=np.int64)
    scored = None if fx["scored"] is None else np.array(fx["scored"], dtype=bool)
    tree = build_tree(flat, cu, scored=scored)
    meta = TreeMeta(tree, "cpu")
    T_tree = len(tree.tokens)
    hidden = (torch.arange(T_tree, dtype=torch.float64) * 0.5 + 1.0)[None, :, None]  # row value of tree row i

    def head(rows, labels):  # (row value + 1000 * label, -label): both columns name the pair
        lab = labels.to(torch.float64)
        return torch.stack([rows[:, 0] + 1000.0 * lab, -lab], -1)

    out = tree_head_output(head, hidden, meta)[0]
    want = _next_token_expectation(flat, cu, scored, tree.flat_to_tree,
                                   lambda pos, nxt: [pos * 0.5 + 1.0 + 1000.0 * nxt, -float(nxt)])
    assert torch.equal(out.to(torch.float64), want)



@pytest.mark.parametrize("k", range(len(NAMES)), ids=NAMES)
def test_bound_head_reproduces_each_familys_softmax(k):
    """The property of reference tests/test_lm_head.py:11-34: once bound, the model returns for each position the
    log-probability of its next token and the entropy of the softmax of its OWN logits (post-head ops included) at
    temperature T, to 1e-5 on the CPU; here the expected columns come from torch.distributions.Categorical over the
    unbound model's logits in fp64, at T 1.0, 0.7 and 1.6. The fused epilogue's reading of each family's recorded
    chain is checked beside it."""
    from transformers import AutoModelForCausalLM
    _, config, (pre, post, tanh) = families()[k]
    torch.manual_seed(40 + k)
    model = AutoModelForCausalLM.from_config(config, attn_implementation="eager")
    model.eval()
    ids = torch.randint(0, config.vocab_size, (1, 15), generator=torch.Generator().manual_seed(50 + k))
    nxt = ids[0].roll(-1)
    with torch.no_grad():
        own = model(input_ids=ids).logits[0].double()
    for temperature in (1.0, 0.7, 1.6):
        head = bind_head(model, temperature)
        head.octopus_labels, head.octopus_tree = nxt, None
        with torch.no_grad():
            cols = model(input_ids=ids).logits[0].double()
        want = torch.distributions.Categorical(logits=own / temperature)
        assert (cols[:, 0] - want.log_prob(nxt)).abs().max().item() <= 1e-5, temperature
        assert (cols[:, 1] - want.entropy()).abs().max().item() <= 1e-5, temperature
    assert (len(head.octopus_post) > 0) == ((pre, post, tanh) != (1.0, 1.0, False))
    fp = _fused_post(head.octopus_post)
    assert abs(fp.pre - pre) < 1e-12 and abs(fp.post - post) < 1e-12 and fp.tanh == tanh


def test_bind_head_binds_each_calls_grpo_inputs():
    """bind_head's pre-hook binds the micro-batch's GRPO inputs from each call's kwargs (advantages, behaviour
    logprobs, loss mask, and proximal logprobs when given) to head.octopus_grpo, flat per position, and None for a call
    without them (compute_logp's batch); binding again replaces the hook. CPU tensors take the composite route with
    the inputs bound: the same columns as without them."""
    from transformers import AutoModelForCausalLM
    _, config, _ = families()[0]
    torch.manual_seed(3)
    model = AutoModelForCausalLM.from_config(config, attn_implementation="eager").eval()
    bind_head(model, 1.0)
    head = bind_head(model, 0.7)
    assert len(model._forward_pre_hooks) == 1
    ids = torch.randint(0, config.vocab_size, (1, 11), generator=torch.Generator().manual_seed(4))
    head.octopus_labels, head.octopus_tree = ids[0].roll(-1), None
    adv, old, mask = torch.randn(1, 11), torch.randn(1, 11), (torch.rand(1, 11) < 0.6).float()
    with torch.no_grad():
        plain = model(input_ids=ids).logits
        assert head.octopus_grpo is None
        bound = model(input_ids=ids, advantages=adv, logprobs=old, loss_mask=mask).logits
    g = head.octopus_grpo
    assert g is not None and g.prox is None and (g.eps_lo, g.eps_hi, g.reject_upper) == (0.2, 0.28, 5.0)
    assert torch.equal(g.adv, adv.reshape(-1)) and torch.equal(g.old, old.reshape(-1))
    assert torch.equal(g.mask, mask.reshape(-1))
    assert torch.equal(plain, bound)
    with torch.no_grad():
        model(input_ids=ids, advantages=adv, logprobs=old, loss_mask=mask, prox_logp=old * 0.5)
    assert torch.equal(head.octopus_grpo.prox, (old * 0.5).reshape(-1))
    with torch.no_grad():
        model(input_ids=ids, advantages=adv, loss_mask=mask)  # no behaviour logprobs: nothing bound
    assert head.octopus_grpo is None


def _llama_with_tail(after_head):
    """A Llama whose forward returns after_head(model, lm_head output) as its logits, with one extra Linear child."""
    from transformers import LlamaConfig
    from transformers.modeling_outputs import CausalLMOutput
    from transformers.models.llama.modeling_llama import LlamaForCausalLM

    class TailedLlama(LlamaForCausalLM):
        def __init__(self, config):
            super().__init__(config)
            self.side = torch.nn.Linear(config.vocab_size, config.vocab_size, bias=False)

        def forward(self, input_ids, **_unused):
            last = self.model(input_ids=input_ids).last_hidden_state
            return CausalLMOutput(logits=after_head(self, self.lm_head(last)))

    torch.manual_seed(7)
    return TailedLlama(LlamaConfig(**TINY))


def _set_first(x):
    x[..., 0] = -1.0
    return x


@pytest.mark.parametrize("after_head", [
    lambda m, x: x.clamp_(min=-4.0),                 # a write into the head's output
    lambda m, x: _set_first(x),                      # an indexed write
    lambda m, x: torch.maximum(x * 2.0, x),          # the flow forks: the earlier result is read again
    lambda m, x: m.side(x),                          # a further submodule
], ids=["inplace", "setitem", "fork", "submodule"])
def test_post_head_flows_one_chain_cannot_replay_are_refused(after_head):
    """The refusals of reference tests/test_lm_head.py:37-55: bind_head raises NotImplementedError for logits that no
    chain of ops on the head's output reproduces."""
    with pytest.raises(NotImplementedError):
        bind_head(_llama_with_tail(after_head), 1.0)


def test_a_replayable_post_head_chain_is_bound_and_fused():
    """A chain of the kinds the fused epilogue takes (a divide, tanh, a multiply) is recorded, read as
    4 tanh(z / 4), and the bound head reproduces the tailed model's own softmax."""
    model = _llama_with_tail(lambda m, x: torch.tanh(x / 4.0) * 4.0).eval()
    ids = torch.randint(0, TINY["vocab_size"], (1, 9), generator=torch.Generator().manual_seed(8))
    with torch.no_grad():
        own = model(input_ids=ids).logits[0].double()
    head = bind_head(model, 0.9)
    assert _fused_post(head.octopus_post) == (0.25, 4.0, True)
    head.octopus_labels, head.octopus_tree = ids[0].roll(-1), None
    with torch.no_grad():
        cols = model(input_ids=ids).logits[0].double()
    want = torch.distributions.Categorical(logits=own / 0.9)
    assert (cols[:, 0] - want.log_prob(ids[0].roll(-1))).abs().max().item() <= 1e-5
    assert (cols[:, 1] - want.entropy()).abs().max().item() <= 1e-5


def test_scored_positions_alone_give_the_same_values_and_gradients():
    """The property of reference tests/test_lm_head.py:58-75 in fp64: with octopus_scored set, the scored positions'
    columns equal those of the unscored head exactly, the others are exactly 0, and the gradient of any loss over the
    scored positions is exactly the same for every parameter (torch.autograd.grad of both runs)."""
    from transformers import AutoModelForCausalLM, LlamaConfig
    torch.manual_seed(11)
    model = AutoModelForCausalLM.from_config(LlamaConfig(**TINY), attn_implementation="eager").to(torch.float64)
    ids = torch.randint(0, TINY["vocab_size"], (1, 14), generator=torch.Generator().manual_seed(12))
    head = bind_head(model, 0.8)
    head.octopus_labels, head.octopus_tree = ids[0].roll(-1), None
    keep = torch.rand(14, generator=torch.Generator().manual_seed(13)) < 0.5
    weight = torch.randn(14, 2, dtype=torch.float64, generator=torch.Generator().manual_seed(14)) * keep[:, None]
    params = list(model.parameters())

    def run(scored):
        head.octopus_scored = scored
        cols = model(input_ids=ids).logits[0]
        return cols.detach(), torch.autograd.grad((cols * weight).sum(), params, allow_unused=True)

    cols_all, grads_all = run(None)
    cols_sel, grads_sel = run(keep)
    assert torch.equal(cols_sel[keep], cols_all[keep]) and bool((cols_sel[~keep] == 0).all())
    for a, b in zip(grads_all, grads_sel):
        assert (a is None and b is None) or torch.equal(a, b)


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
        # with the trainer's own seq_tiles module loaded, its flag (the one its decoder layers read) follows too
        import sys
        import types
        ref = types.ModuleType("octopus.rl.seq_tiles")
        ref._INNER = True
        sys.modules["octopus.rl.seq_tiles"] = ref
        try:
            with seq_tiles.no_inner():
                assert ref._INNER is False and seq_tiles._INNER is False
            assert ref._INNER is True
        finally:
            del sys.modules["octopus.rl.seq_tiles"]
        a, b = seq_tiles.tiled(lambda p, q: (p + 1, q), x, None if False else x)
        assert a.shape == x.shape and torch.equal(b, x)
    finally:
        seq_tiles.TILE = old


def test_prefix_tree_module_exports():
    assert callable(prefix_tree.build_tree) and callable(prefix_tree.tree_head_output)


def test_the_head_op_saves_no_weight_for_backward():
    """An activation-offload pack hook (saved_tensors_hooks, as the actor's host_activations) sees the rows, labels and
    per-row state the head op saves, never the [V, d] weight: the backward reads the weight the op holds by reference
    (meta tensors through the op's fake kernels; no GPU). The backward still returns a [V, d] weight gradient."""
    from octopus_amd import head_op
    V, d, n = 1000, 64, 32
    rows = torch.empty(n, d, device="meta", dtype=torch.bfloat16, requires_grad=True)
    W = torch.empty(V, d, device="meta", dtype=torch.bfloat16, requires_grad=True)
    labels = torch.empty(n, device="meta", dtype=torch.int64)
    packed = []

    def pack(t):
        packed.append(tuple(t.shape))
        return t

    with torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t):
        out = head_op.fused_head(rows, W, labels, 0.9)
    assert packed and (V, d) not in packed, packed
    out[:, 0].sum().backward()
    assert W.grad.shape == (V, d) and rows.grad.shape == (n, d)


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


def test_the_fused_step_saves_no_weight_gradient_for_backward():
    """The fused GRPO step computes both gradients in its forward call and holds them for the backward on the autograd
    context, out of a pack hook's reach: saved_tensors_hooks sees no [V, d] tensor (meta tensors through the op's fake
    kernels; no GPU), and loss.backward() still gives rows and weight their gradients."""
    from octopus_amd import head_op
    V, d, n = 1000, 64, 32
    rows = torch.empty(n, d, device="meta", dtype=torch.bfloat16, requires_grad=True)
    W = torch.empty(V, d, device="meta", dtype=torch.bfloat16, requires_grad=True)
    labels = torch.empty(n, device="meta", dtype=torch.int64)
    adv = torch.empty(n, device="meta", dtype=torch.float32)
    mask = torch.empty(n, device="meta", dtype=torch.bool)
    packed = []

    def pack(t):
        packed.append(tuple(t.shape))
        return t

    with torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t):
        loss, out = head_op.fused_grpo_head(rows, W, labels, 0.9, adv, mask)
    assert (V, d) not in packed and (n, d) not in packed, packed
    assert out.shape == (n, 2) and not out.requires_grad
    loss.backward()
    assert W.grad.shape == (V, d) and rows.grad.shape == (n, d)
