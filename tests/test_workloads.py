"""The seeded workloads match the configurations they stand for: packed-token totals, scored rows, and the tree
shapes (root, branches, depth, fan-out, node sizes) their descriptions give."""

import pytest

from octopus_amd.workloads import CFG4_INNER, CONFIGS


def _scored(cfg):
    return sum(n for n, s, _ in cfg.segments if s)


@pytest.mark.parametrize("name,N,scored", [("cfg1", 512, 512), ("cfg2", 32768, 32768), ("cfg3", 32768, 24576),
                                           ("cfg5", 131072, 114688)])
def test_packed_and_scored_tokens(name, N, scored):
    cfg = CONFIGS[name]
    assert sum(n for n, _, _ in cfg.segments) == cfg.N == N
    assert _scored(cfg) == scored


def test_cfg4_is_a_depth_3_fan_out_4_dag_with_about_55_percent_masked():
    """Root of 4,096 tokens, then pre-order: each shared node is followed by its 4 children, leaves (scored) of
    U[1024, 4096] tokens, shared nodes (masked) of CFG4_INNER tokens, laid out until 65,536 tokens with the last one
    trimmed; the masked share is about 55% (56.2% at seed 5)."""
    segs = CONFIGS["cfg4"].segments
    assert sum(n for n, _, _ in segs) == 65536
    assert segs[0][:2] == (4096, False)
    # walk the pre-order list: a masked node opens 4 children at the next depth
    stack = [(0, 4)]  # (depth of the node whose children come next, children left)
    for i, (n, scored, _) in enumerate(segs[1:], start=1):
        parent_depth, left = stack[-1]
        d = parent_depth + 1
        last = i == len(segs) - 1
        if d == 3:
            assert scored and (1024 <= n <= 4096 or last)
        else:
            assert not scored and (n == CFG4_INNER or last)
        stack[-1] = (parent_depth, left - 1)
        if not scored:
            stack.append((d, 4))
        while stack and stack[-1][1] == 0:
            stack.pop()
    masked = 1 - _scored(CONFIGS["cfg4"]) / 65536
    assert 0.52 <= masked <= 0.58, masked
    assert _scored(CONFIGS["cfg4"]) == 28672
