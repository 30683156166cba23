"""Shared helpers for the parity tests: seeded inputs and tolerance checks."""
from __future__ import annotations

import numpy as np

from oracle import oracle as o


def normal(count: int, seed: int, stream: int = 0, scale: float = 1.0) -> np.ndarray:
    """Seeded N(0,1) values (mulberry32 + Box-Muller, oracle implementation)."""
    return o.normal(count, seed, stream, scale)


def quantized_matrix(fmt: int, rows: int, cols: int, seed: int, stream: int = 0, scale: float = 0.02):
    values = normal(rows * cols, seed, stream, scale).reshape(rows, cols)
    scales, data = o.quantize_rows(fmt, values)
    return values, scales, data


def assert_close(actual, expected, rtol: float = 1e-3, atol_rms: float = 1e-3, what: str = ""):
    """|a - r| <= rtol |r| + atol_rms * rms(r): relative error, with the
    output's own scale as the floor for values near zero."""
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    assert actual.shape == expected.shape, (actual.shape, expected.shape)
    rms = float(np.sqrt(np.mean(expected ** 2))) if expected.size else 0.0
    bound = rtol * np.abs(expected) + atol_rms * max(rms, 1e-30)
    err = np.abs(actual - expected)
    bad = err > bound
    if bad.any():
        i = int(np.argmax(err - bound))
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {err.size} outside tolerance; worst index {i}: "
            f"actual {actual.flat[i]!r} expected {expected.flat[i]!r} (max abs err {err.max():.3e}, rms {rms:.3e})")
    return float((err / np.maximum(np.abs(expected) + rms, 1e-30)).max()) if err.size else 0.0


def lcg_values(count: int, state: int, divisor: float):
    """kernels.zig:791-803: state = state * 1664525 + 1013904223 (u32),
    value = f32(((state >> 9) % 2001) - 1000) / divisor."""
    out = np.zeros(count, np.float32)
    for i in range(count):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32(((state >> 9) % 2001) - 1000) / np.float32(divisor)
    return out, state


# Norm vector kinds (QWH_T_* / the oracle's QWREF_VEC_*).
ATTN_NORM, Q_NORM, K_NORM, FFN_NORM, FINAL_NORM = 16, 17, 18, 19, 20


def random_norms(config: dict, seed: int) -> dict:
    """Norm weight vectors with distinct entries around 1, as a real
    checkpoint's learned RMSNorm weights: per layer attention, q, k and ffn,
    plus the final norm."""
    hidden, head_dim = config["hidden"], config["head_dim"]
    out = {"final": 1.0 + 0.5 * normal(hidden, seed, 900)}
    for layer in range(config["layers"]):
        out[layer] = dict(attn=1.0 + 0.5 * normal(hidden, seed, 901 + 8 * layer),
                          q=1.0 + 0.5 * normal(head_dim, seed, 902 + 8 * layer),
                          k=1.0 + 0.5 * normal(head_dim, seed, 903 + 8 * layer),
                          ffn=1.0 + 0.5 * normal(hidden, seed, 904 + 8 * layer))
    return out


def set_norms(decoder, norms: dict, layers: int) -> None:
    """Binds random_norms() vectors on an oracle or a device decoder (both
    take set_vector(kind, layer, values))."""
    decoder.set_vector(FINAL_NORM, 0, norms["final"])
    for layer in range(layers):
        n = norms[layer]
        decoder.set_vector(ATTN_NORM, layer, n["attn"])
        decoder.set_vector(Q_NORM, layer, n["q"])
        decoder.set_vector(K_NORM, layer, n["k"])
        decoder.set_vector(FFN_NORM, layer, n["ffn"])
