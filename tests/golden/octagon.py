"""Reader for the Octagon text fixtures (``Type { Field: [..] ... }``)."""
import re
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent


def load(name: str) -> dict:
    text = (GOLDEN / name).read_text()
    fields = {}
    for m in re.finditer(r"(\w+):\s*\[([^\]]*)\]", text):
        values = [v for v in m.group(1 + 1).replace("\n", " ").split(",") if v.strip()]
        fields[m.group(1)] = np.array([float(v) for v in values], dtype=np.float64)
    return fields
