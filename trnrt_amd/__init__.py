"""trnrt_amd: an MI355X (gfx950) implementation of TrnRT's DSA decode path behind TrnRT's operator surface.

The three operators of a DeepSeek-Sparse-Attention decode layer (lightning indexer, exact top-k, sparse MLA over a
paged FP8 KV cache) run as hand-written HIP kernels in libdsa_gfx950.so, reached through ctypes. The modules keep the
reference's names: trnrt_amd.kernels.dsa_index / dsa_topk / dsa_decode / dsa_slots_n and
trnrt_amd.models.dsa_long mirror trnrt.kernels.* and trnrt.models.dsa_long.
"""

__version__ = "0.1.0"
