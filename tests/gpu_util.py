"""Helpers shared by the GPU parity tests (not collected by pytest)."""
import numpy as np


def rel_err(got, ref):
    """max|got - ref| / RMS(ref): the parity metric of the layer."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    rms = np.sqrt(np.mean(ref ** 2))
    return float(np.max(np.abs(got - ref)) / (rms + 1e-300))


def to_np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def print_case(**kw):
    """Name the case before a GPU step so a crash report points at it."""
    print("CASE " + " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def bf16_excess_err(got, ref):
    """Error of a bf16 output beyond its own final rounding, relative to RMS(ref).

    A bf16 result differs from the exact value by up to half an ulp
    (2^-9 |ref|) from the store alone; the 5e-3 bf16 bar applies to what is
    left after that: max(|got - ref| - 2^-8 |ref|, 0) / RMS(ref), which
    allows one rounding step either way.
    """
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    rms = np.sqrt(np.mean(ref ** 2))
    excess = np.maximum(np.abs(got - ref) - 2.0 ** -8 * np.abs(ref), 0.0)
    return float(np.max(excess) / (rms + 1e-300))
