"""undertow_amd: MI355X (gfx950) backend of undertow's MTP draft+verify step.

The product is ``lib/libundertow_hip.so`` (hand-written HIP behind the C ABI
in ``include/undertow_hip.h``); this package is its host-side binding.
"""
from .runtime import (  # noqa: F401
    EXPORTED, F32, INFER, INT4, INT8, LIB_PATH, LRU, WEIGHTED, Context, ContextOverflow,
    ExpertProfile, ExpertTable, Model, StoreConfig, StoreStats,
    ModelConfig, QTensor, Session, ShapeError, UtError, argmax_rows, lib, mla_attend,
    mla_attend_split, mla_cache_split, route,
)
