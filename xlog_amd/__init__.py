"""xlog_amd — MI355X-native (gfx950) relational core for XLOG's semi-naive fixpoint.

The product is libxlog_hip.so (HIP kernels + C ABI, include/xlog_hip.h);
`xlog_amd.provider` mirrors the reference's CudaKernelProvider on top of it.
"""
from .provider import (  # noqa: F401
    HipKernelProvider,
    Relation,
    JoinIndex,
    FjDeltaCols,
    FJ_DELTA_CANONICAL,
    XlogError,
    JOIN_INNER,
    JOIN_SEMI,
    JOIN_ANTI,
    ROUTE_AUTO,
    ROUTE_JOIN,
    ROUTE_BITMAP,
    ROUTE_HASH,
    tc_plan,
    andersen_plan,
    copy_points_to_plan,
    pack,
    unpack,
    arrow_ipc_decode_u32,
    arrow_ipc_encode_u32,
    library_path,
    ABI_SYMBOLS,
)

__version__ = "0.1.0"
