"""MI355X-native nested Gated DeltaNet chunkwise memory op.

Drop-in for ``nested_gdn2.ops.chunk_nested_gdn2`` of awehrs/nested_recurrent_memory
and for its decoding step ``naive_step_nested_gdn2``, computed by hand-written
gfx950 HIP kernels (libngdn.so, C ABI in include/ngdn.h), and the layer around
them (``NestedGDN2Attention``) with fla's two modules replaced by kernels of
the same library.
"""

from .chunk import PROMOTIONS, ChunkNestedGDN2Function, chunk_nested_gdn2
from .layer import NestedGDN2Attention, NestedGDN2LayerConfig
from .layer_ops import FusedRMSNormGated, ShortConvolution
from .schedule import n_firings, n_groups, source_index
from .step import prepare_step_params, step_nested_gdn2

__all__ = ["chunk_nested_gdn2", "ChunkNestedGDN2Function", "PROMOTIONS",
           "step_nested_gdn2", "prepare_step_params", "n_firings", "n_groups", "source_index",
           "NestedGDN2Attention", "NestedGDN2LayerConfig", "ShortConvolution", "FusedRMSNormGated"]
