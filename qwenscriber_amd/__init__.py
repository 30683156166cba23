"""MI355X (gfx950) backend for Qwenscriber's quantized decoder hot path.

The product is the C-ABI library ``qwenscriber_amd/build/libqwhip.so``
(``include/qwhip.h``). This module is a thin ctypes binding for Python callers
(tests, benchmarks): every call goes to the HIP library, and importing the
binding fails loudly when the library is not built -- there is no CPU path.
"""
from __future__ import annotations

from ._lib import (  # noqa: F401
    DATA_BYTES,
    FORMAT_Q4,
    FORMAT_Q5,
    FORMAT_Q8,
    GROUP_SIZE,
    AudioLayerWeights,
    Context,
    Decoder,
    DecoderConfig,
    DeviceBuffer,
    ModelConfig,
    QwhError,
    TensorEntry,
    config_decoder,
    config_parse,
    library_path,
    load,
    shard_find,
    shard_validate,
    shard_verify_checksum,
)
