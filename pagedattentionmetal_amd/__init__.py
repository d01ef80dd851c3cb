"""pagedattentionmetal_amd - PagedAttentionMetal's ragged paged-attention path on MI355X.

The work happens in ``libpam.so`` (hand-written gfx950 HIP kernels + C++ runtime
behind the reference's ``pam_*`` C ABI, declared in ``include/pam.h``).  This
package mirrors the reference's Swift API over that ABI.
"""
from .api import (BlockEvictionPolicy, ContinuousBatchingScheduler, KVCacheManager, PagedAttentionDataType,
                  PagedAttentionEngine, PagedAttentionError, PagedLayerSpec, SequenceStatus)

__all__ = ["BlockEvictionPolicy", "ContinuousBatchingScheduler", "KVCacheManager", "PagedAttentionDataType",
           "PagedAttentionEngine", "PagedAttentionError", "PagedLayerSpec", "SequenceStatus"]
