"""MI355X-native KV-cache data path with the API of rouviere-german/paged-kv-serving.

The K/V pool lives in HBM; the slot-mapped append, the copy-on-write block copy and paged
attention over block tables (decode and chunked-prefill rows in one ragged call) are
hand-written HIP kernels for gfx950 in ``csrc/``, exported through the C ABI of
``include/pkv.h`` as ``libpkv.so`` and called through ``ctypes``. The host side keeps the
reference's Python API:

    runner        ModelRunner, BatchEntry, ExecutionBatch   (reference engine/runner.py)
    blocks        BlockManager, BlockStore, errors          (reference engine/blocks.py)
    kvcache       KVCacheManager                            (reference engine/kvcache.py)
    prefix_cache  PrefixCache and the block hash chain      (reference engine/prefix_cache.py)
    attention     paged_attention                           (reference engine/attention.py)
    equivalence   paged vs cache-free logits on the device  (reference engine/equivalence.py)
    replay        a recorded reference serving run driven through the KV-cache manager and runner
    ops           tensor-level calls into libpkv.so
    workloads     seeded synthetic batches of the benchmark configurations

Modules that touch the device import torch; ``blocks``, ``kvcache``, ``prefix_cache``,
``sequence``, ``config`` and ``model`` are plain Python/NumPy.
"""

__version__ = "0.1.0"
