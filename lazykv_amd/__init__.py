"""lazykv_amd: LazyKV's tiered decode-attention hot path, native on MI355X (gfx950).

The kernels live in `csrc/` (hand-written HIP) behind the C ABI of `include/lazykv_hip.h`, built
in-tree into `liblazykv_hip.so`. The Python modules keep the call surface of the reference's
modules: `selection` (quest_bound, top_blocks), `quant` (pack, unpack), `exact` (merge_lse,
partial attention), `pinned` (pinned_empty, device_view), `attention` (the registered attention
function) and `tiered` (TieredLayer, TieredCache, ExactTieredCache).
"""

__all__ = ["attention", "exact", "kernels", "pinned", "quant", "selection", "tiered"]
