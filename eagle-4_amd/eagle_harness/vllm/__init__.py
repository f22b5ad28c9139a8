"""Engine-side pieces of the vLLM adapter on the verify hot path: the tree-verify attention and its CUSTOM backend, the
verify stage (tree masks, depths, window codes), the greedy tree walk, the GDN / Mamba2 layer hook with the
accepted-path state commit, and the round commit that puts a tree round back into chain order (KV compaction,
chainize).

The rest of the vLLM plugin (registration, the speculator, the draft model, configuration) is the installed
eagle-harness's: this package's ``__path__`` continues into it."""

from pkgutil import extend_path

__path__ = extend_path(__path__, __name__)
