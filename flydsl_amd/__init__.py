"""flydsl_amd -- MI355X-native (gfx950) FP8-KV paged-attention decode.

Drop-in host API with the signatures of the reference modules
kernels/pa_decode_fp8.py, kernels/pa_decode_swa.py and kernels/pa_metadata.py,
backed by hand-written HIP kernels in libpa_fp8.so (C ABI: include/pa_fp8.h).
"""

from .pa_decode_fp8 import (  # noqa: F401
    KV_COMPUTE_BLOCK,
    get_pa_metadata,
    get_recommended_splits,
    pa_decode_ps_launch,
)
from .pa_decode_swa import get_sw_max_context_partition_num, pa_decode_sw_reduce  # noqa: F401
from .pa_metadata import get_pa_metadata_info_v1, get_pa_metadata_v1  # noqa: F401
from .pa_reduce import pa_reduce_v1  # noqa: F401

__all__ = [
    "KV_COMPUTE_BLOCK",
    "get_pa_metadata",
    "get_pa_metadata_info_v1",
    "get_pa_metadata_v1",
    "get_recommended_splits",
    "get_sw_max_context_partition_num",
    "pa_decode_ps_launch",
    "pa_decode_sw_reduce",
    "pa_reduce_v1",
]
