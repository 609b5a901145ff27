"""jinf_amd: MI355X (gfx950) kernels for jinf's per-layer elementwise and
reduction path -- RMSNorm (+ fused residual add), interleaved GQA RoPE,
SwiGLU, masked row softmax and the GGUF Q4_0 token-embedding gather -- and,
beside them, the dequant-GEMV and row dequant for GGUF Q4_0 / Q8_0 / Q4_K /
Q6_K weights, GQA decode attention, GGUF and .nvmw model files and the
decode engine that runs them all per token.

The kernels live in libjinf_hip.so behind the C-ABI of include/jinf/*.h;
this package is a thin ctypes/torch front end used by tests and bench.py.
"""
from ._lib import F16, F32, LIB_PATH, Q4_0, Q4_K, Q6_K, Q8_0, lib, version  # noqa: F401
from .ops import (  # noqa: F401
    JinfError,
    attention_decode,
    attention_workspace,
    cuda_attention,
    cuda_dequant_matvec,
    cuda_dequantize,
    cuda_dequantize_q4_0,
    cuda_residual_add,
    cuda_rmsnorm,
    cuda_rope,
    cuda_silu_mul,
    cuda_softmax,
    dequant_rows,
    embed_q4_0,
    matvec,
    matvec_add,
    matvec_batch,
    matvec_batch_add,
    matvec_batch_workspace,
    matvec_q4_0,
    residual_add,
    residual_rmsnorm_rows,
    rmsnorm_matvec,
    rmsnorm_matvec_batch,
    rmsnorm_qkv_rope,
    rmsnorm_qkv_rope_batch,
    rmsnorm_rows,
    rmsnorm_swiglu_matvec,
    rmsnorm_swiglu_matvec_batch,
    rope_rows,
    softmax_rows,
    swiglu,
)
from . import gguf  # noqa: F401,E402
from . import nvmw  # noqa: F401,E402
from .engine import Batch, Engine, EngineError  # noqa: F401,E402
