"""Mirror of the reference trainer's LM-head modules (octopus/rl/lm_head.py, prefix_tree.py, seq_tiles.py)."""
