"""rce_amd -- MI355X (gfx950) GGUF block-quantized matmul path.

The product is the C-ABI library ``rce_amd/lib/librce_qmm.so`` (HIP kernels
in ``rce_amd/csrc``, interface ``include/rce_qmm.h``).  ``rce_amd.qmm`` is the
Python mirror of the reference operator API (``rce-op-qmm``) over that ABI;
``rce_amd.llama`` mirrors the TinyLlama decode runtime (``rce-tinyllama``);
``rce_amd.gguf`` the GGUF file reader (``rce-ingest-gguf``).
"""
from .qmm import (  # noqa: F401
    NOALLOC_SCRATCH_BYTES, Context, DeviceBuffer, GgufDtype, Mode, QmmError, QuantWeight, block_geometry, mm_1d,
    mm_1d_serial, mm_batched, mm_batched_dev, mm_batched_dev_noalloc, moe_ffn_dev, moe_router, moe_swiglu_dev,
    quantize, row_bytes, supports,
)
from .llama import TinyLlamaBlock, TinyLlamaConfig, TinyLlamaRuntime, TinyLlamaWeights, load_weights  # noqa: F401,E402
from .gguf import GgufFile, GgufMetadata, GgufTensorInfo, GgufValue, split_experts  # noqa: F401,E402
from .placement import (GpuEnergyMeter, HipQmm, HostQuantWeight, LinearCoeffs, hip_cost_prior,  # noqa: F401,E402
                        pick_priced, qmm_dtype_id)
