"""The oracle: a CPU restatement of the reference's LM-head path, used ONLY as the checker.

Test infrastructure. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import it; the
product (octopus_amd) never does, and nothing here runs on or feeds the GPU path.

    oracle.head      per-row logprob / entropy / lse and the closed-form backward, fp64 (torch on CPU)
    oracle.pairs     masked-row compaction and the (tree position, label) pair section (numpy / Python)
    oracle.grpo      the GRPO objective's per-token weight g = dL/dlogp (numpy, fp64)
    oracle.baseline  the reference algorithm as the reference runs it (CHUNK-row chunks, input-dtype GEMM,
                     fp32 softmax, checkpointed backward) for the timed CPU baseline

Pinning (tests/test_oracle.py): every function is checked against something other than its own formula —
transformers' model logits with torch.log_softmax, brute-force Python loops, closed-form special cases,
finite differences, torch autograd, torch.nonzero, and the reference's hand-built test cases
(tests/test_lm_head.py, tests/test_prefix_tree.py of the reference).
"""
