"""Loading helpers for the golden fixtures in tests/golden/."""
import json
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name: str):
    data = np.load(GOLDEN / (name + ".npz"), allow_pickle=False)
    meta_path = GOLDEN / (name + ".json")
    meta = json.loads(meta_path.read_text()) if meta_path.exists() else None
    return data, meta
