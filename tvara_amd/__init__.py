"""MI355X-native paged KV cache and paged attention for Tvara.

The compute path is libtvara_capi.so (hand-written HIP for gfx950, C ABI in
include/tvara_capi.h); this package is its Python surface:

* tvara_amd.kv         -- PagedCache / BlockPool over HBM (core/include/tvara/kv.hpp)
* tvara_amd.attention  -- fused paged decode and causal prompt attention
                          (core/include/tvara/attention.hpp)
* tvara_amd.workloads  -- the synthetic workloads of the benchmarks and tests
* tvara_amd.build      -- the in-tree hipcc build
"""

__all__ = ["kv", "attention", "synth", "workloads"]
