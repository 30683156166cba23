"""MI355X (gfx950) backend for Qwenscriber's quantized decoder hot path.

The product is the C-ABI library ``qwenscriber_amd/build/libqwhip.so``
(``include/qwhip.h``). This module is a thin ctypes binding for Python callers
(tests, benchmarks): every call goes to the HIP library, and importing the
binding fails loudly when the library is not built -- there is no CPU path.
"""
from __future__ import annotations

from ._lib import (  # noqa: F401
    CACHE_F32,
    CACHE_Q8,
    DATA_BYTES,
    FORMAT_F16,
    FORMAT_F32,
    FORMAT_Q4,
    FORMAT_Q5,
    FORMAT_Q8,
    GROUP_SIZE,
    AudioFrontendWeights,
    AudioLayerWeights,
    Context,
    Decoder,
    DecoderConfig,
    DeviceBuffer,
    ModelConfig,
    QwhError,
    T_ATTN_NORM,
    T_DOWN,
    T_EMBED,
    T_FFN_NORM,
    T_FINAL_NORM,
    T_GATE,
    T_K,
    T_K_NORM,
    T_LM_HEAD,
    T_O,
    T_Q,
    T_Q_NORM,
    T_UP,
    T_V,
    TensorEntry,
    config_decoder,
    config_parse,
    library_path,
    load,
    shard_find,
    shard_validate,
    shard_verify_checksum,
)
