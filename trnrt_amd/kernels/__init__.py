"""The DSA operator surface of trnrt/kernels (dsa_index, dsa_topk, dsa_decode, dsa_slots_n) on gfx950, plus the
whole decode layer in one call (dsa_layer)."""
