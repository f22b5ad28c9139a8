"""Engine-free pieces of the reference's vLLM adapter that sit on the verify hot path: the tree-verify attention,
the verify stage (tree masks, depths, window codes), the greedy tree walk, the accepted-path state commit, and the
round commit that puts a tree round back into chain order (KV compaction, chainize)."""
