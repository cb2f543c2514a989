"""purebee_amd -- MI355X (gfx950) backend for PureBee's quantized matmul instruction.

The product is the C ABI of ``include/pbx.h`` (``lib/libpbhip.so``, which loads
the gfx950 code objects ``lib/*.hsaco`` with hipModuleLoad), the N-API addon
``lib/pbx_napi.node`` and the JavaScript drop-in modules under ``js/``.
:mod:`purebee_amd.native` is a thin ctypes binding of the same C ABI for
Python callers (tests, bench).
"""
from .native import (  # noqa: F401
    PbxError, Context, Weight, Model, ModelConfig, GGUF, load_library, library_path,
    TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q4_1, TYPE_Q8_0, TYPE_Q6_K, TYPE_Q8_REF, row_bytes,
    quantize_q4_0, quantize_q4_1, quantize_q6_k, quantize_q8_0, to_f16_bytes, quantize_q8_ref, synth_normal, block_bytes,
    speculative_generate,
)
