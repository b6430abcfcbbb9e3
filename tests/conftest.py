import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "tgtts-v4_amd", ROOT / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def ctx():
    """The GPU context, one per session (the process's only one)."""
    import tgx

    c = tgx.Context(0)
    report = c.report()
    print(f"\n[gpu] {report['name']} {report['arch']} CUs {report['compute_units']} clock {report['clock_khz']} kHz", flush=True)
    yield c
    c.close()


def distance(got: np.ndarray, want: np.ndarray) -> dict:
    """The reference's Distance (crates/graph/tests/decode.rs:52-90), plus cosine and
    max|got - want| / max|want|."""
    g = np.asarray(got, dtype=np.float64).ravel()
    w = np.asarray(want, dtype=np.float64).ravel()
    d = np.abs(g - w)
    max_abs = float(np.max(d)) if np.all(np.isfinite(d)) else float("inf")
    rel_rms = float(np.sqrt(np.sum(d * d) / np.sum(w * w)))
    cos = float(np.dot(g, w) / (np.linalg.norm(g) * np.linalg.norm(w)))
    rel_max = max_abs / float(np.max(np.abs(w)))
    return {"max_abs": max_abs, "relative_rms": rel_rms, "cosine": cos, "rel_max": rel_max}


# The accuracy bar for bf16 on the GPU against the fp64 oracle over the same bf16 weights:
# cosine >= 0.999 and max|got - ref| / max|ref| <= 1e-2, per step.
COSINE_MIN = 0.999
REL_MAX = 1e-2


def within(d: dict) -> bool:
    return d["cosine"] >= COSINE_MIN and d["rel_max"] <= REL_MAX
