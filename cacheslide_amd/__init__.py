"""MI355X-native CacheSlide reuse-attention hot path.

Drop-in counterparts of the reference's cacheslide_vllm modules for CCPE
attention (position, attention), WCA (wca, policy) and SLIDE slot management
(slide, paged), computing on hand-written gfx950 kernels in
_lib/libcacheslide_hip.so; plus fused paged-cache entry points (ccpe),
batched relocation (relocate), the CCPE profile artifacts (profiles), and
the layer snapshot pages between a page store and HBM (pagestore,
snapshot).
"""

from .attention import CanonicalPositionPolicy, SelectedAssociationPolicy
from .contracts import RequestPlan
from .paged import NativePagedKV
from .policy import WCAConfig
from .position import (
    CCPEPositionError,
    CCPEProfile,
    ChunkIdentity,
    CoPE,
    CoPEPositionTrace,
    cope_attention,
    validate_contextual_path,
)
from .slide import LayerSlotMap, SlotWrite, coalesce_slot_writes
from .snapshot import LayerSnapshots, SnapshotUploader, encode_snapshot, parse_snapshot
from .errors import CacheCapacityError, CacheIntegrityError, StaleCompletionError
from .pagestore import PageStore
from .wca import (
    WCANumericalError,
    WCAState,
    WCAUpdate,
    adaptation_weight,
    mean_head_cosine,
    squared_deviation,
)

__version__ = "0.1.0"

__all__ = [
    "CCPEPositionError", "CCPEProfile", "CacheCapacityError", "CacheIntegrityError",
    "CanonicalPositionPolicy", "ChunkIdentity", "CoPE",
    "CoPEPositionTrace", "LayerSlotMap", "LayerSnapshots", "NativePagedKV", "RequestPlan",
    "PageStore", "SelectedAssociationPolicy", "SlotWrite", "SnapshotUploader",
    "StaleCompletionError", "WCAConfig",
    "WCANumericalError", "WCAState", "WCAUpdate", "adaptation_weight", "coalesce_slot_writes",
    "cope_attention", "encode_snapshot", "mean_head_cosine", "parse_snapshot", "squared_deviation", "validate_contextual_path",
]
