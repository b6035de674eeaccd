"""Reader for the Octagon text fixtures: ``Type { Field: [..]  Field: Sub { A: x B: y }  Field: x }``.

Arrays become float64 numpy arrays; scalars inside nested records are keyed
``Record.Field`` (e.g. ``QNormPair.Even``); scalars of the outer record keep
their own name (e.g. ``Expected``)."""
import re
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent
_NUM = r"-?\d+(?:\.\d*)?(?:[eE][-+]?\d+)?"


def load(name: str) -> dict:
    text = (GOLDEN / name).read_text()
    fields = {}
    for m in re.finditer(r"(\w+):\s*\[([^\]]*)\]", text):
        values = [v for v in m.group(2).replace("\n", " ").split(",") if v.strip()]
        fields[m.group(1)] = np.array([float(v) for v in values], dtype=np.float64)
    for m in re.finditer(r"(\w+):\s*\w+\s*\{([^{}]*)\}", text):
        for s in re.finditer(rf"(\w+):\s*({_NUM})", m.group(2)):
            fields[f"{m.group(1)}.{s.group(1)}"] = float(s.group(2))
    # outer-record scalars: the body with arrays and nested records removed
    body = text[text.index("{") + 1:text.rindex("}")]
    body = re.sub(r"\[[^\]]*\]", "[]", body)
    body = re.sub(r"\w+\s*\{[^{}]*\}", "{}", body)
    for s in re.finditer(rf"(\w+):\s*({_NUM})(?![\w.])", body):
        fields[s.group(1)] = float(s.group(2))
    return fields
