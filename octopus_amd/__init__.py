"""octopus_amd: the chunked LM-head logprob path of Prefix-Tree Packed DAG-GRPO (shatianming5/octopus),
built for MI355X (gfx950) as hand-written HIP kernels behind a C ABI (libocto_head.so), PyTorch custom ops
(octopus_amd.head_op) and the reference's Python call surface (octopus_amd.rl.lm_head, .prefix_tree,
.seq_tiles)."""

__version__ = "0.1.0"
