"""MI355X (gfx950) native implementation of the dotsnote FP8 sparse-MLA attention path.

kernels      tensor wrappers of the C-ABI library libspmla_gfx950.so (include/spmla.h)
sparse_offload  LayerOffload: host-row pool, HBM hot-row cache, store / gather / attend (tiered, split-K, merge)
dsa          PortableSparseImpl / PortableSparseBackend: the vLLM attention-backend surface of the path
shard_indexer, fast_topk  indexer key store, logits and exact top-k
"""
__version__ = "0.1.0"
