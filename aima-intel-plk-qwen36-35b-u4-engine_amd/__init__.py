"""MI355X-native U4 MoE expert hot path (batch-1 decode + grouped prefill).

Hand-written HIP kernels for gfx950 in ``csrc/`` are built into
``libaima_u4moe.so`` behind the C ABI of ``include/aima_u4moe.h``; this
package is the thin host layer over it.  The package directory name is not a
Python identifier, so it is imported under the name ``aima_u4moe``
(``__graft_entry__.load_package()`` registers it).
"""

from . import _lib, layout, ops, runtime, synth  # noqa: F401
from ._lib import AimaError  # noqa: F401
from .layout import MoeLayerWeights, U4Weight  # noqa: F401
from .ops import (  # noqa: F401
    MIN_WEIGHT_SUM,
    DecodePlan,
    DecodeRoutes,
    Qwen36MoeFfnLayerResult,
    RouterTopKSelection,
    Workspace,
    apply_rms_norm,
    build_grouped_schedule,
    ffn_layer_trace,
    grouped_moe_prefill,
    grouped_moe_prefill_routed,
    lm_head_topk,
    matvec_u4,
    matvec_u4_multi,
    moe_decode_down,
    moe_3gemm_fused_compressed,
    moe_decode_gate_up,
    moe_stack_decode,
    moe_stack_decode_routed,
    moe_stack_prefill,
    prefill_workspace_views,
    q4k_unpack,
    q4s_matvec,
    router_fc_topk,
    router_gemm_topk,
    run_moe_ffn_layer,
    select_router_topk,
    topk_f32,
    u4_dequant,
    u4_dequant_f16,
    u4_group_major_to_rows,
    u4_rows_to_group_major,
)
from .runtime import (  # noqa: F401
    GroupedU4PrefillInput,
    GroupedU4PrefillRun,
    GroupedU4PrefillRuntime,
)
