"""Writer of Oct's ``.octagon`` text values, as the reference's interpreter
writes them (internal/interpret/octagon_emit.go:11-130).

The SGEMM corpus report and the async validation record of
``oct_amd.runtime`` are written with it (runtime.go:382-425, 521-566), so a
tool that reads the reference's reports reads these unchanged.  Values:
``bool``, ``int``, ``float``, ``str``, lists (arrays) and ``Record``; the
reference's matrices, vectors, enums and unit suffixes do not occur in these
reports.

Format (octagon_emit.go:34-130): an int in decimal; a float as Go's
``strconv.FormatFloat(v, 'g', -1, 64)`` with ``.0`` appended when that has no
``.``, ``e`` or ``E``; a bool as ``true``/``false``; a string as Go's
``strconv.Quote``; an array as ``[a, b]``; a record as ``Type {`` then one
``    Field: value`` line per field at one more indent (four spaces per level;
int and float fields in parentheses), then ``}`` at the record's own indent.
A written file ends with one newline.
"""
from __future__ import annotations

import math
import os
import unicodedata
from dataclasses import dataclass, field
from decimal import Decimal
from typing import List, Tuple, Union

Value = Union[bool, int, float, str, list, "Record"]


@dataclass
class Record:
    type_name: str
    fields: List[Tuple[str, "Value"]] = field(default_factory=list)


def format_float_g(v: float) -> str:
    """Go's strconv.FormatFloat(v, 'g', -1, 64): the shortest digits that
    round-trip, in %e form when the decimal exponent is below -4 or at least
    6 (shortest 'g' decides with precision 6), else in %f form."""
    if math.isnan(v):
        return "NaN"
    if math.isinf(v):
        return "+Inf" if v > 0 else "-Inf"
    sign = "-" if math.copysign(1.0, v) < 0 else ""
    if v == 0.0:
        return sign + "0"
    t = Decimal(repr(abs(v))).normalize().as_tuple()  # repr: shortest round-trip digits
    digits = "".join(map(str, t.digits))
    dp = len(digits) + t.exponent  # position of the decimal point
    exp = dp - 1
    if exp < -4 or exp >= 6:
        mant = digits[0] + ("." + digits[1:] if len(digits) > 1 else "")
        return f"{sign}{mant}e{'-' if exp < 0 else '+'}{abs(exp):02d}"
    if dp <= 0:
        return f"{sign}0.{'0' * -dp}{digits}"
    if dp >= len(digits):
        return sign + digits + "0" * (dp - len(digits))
    return f"{sign}{digits[:dp]}.{digits[dp:]}"


_ESCAPES = {"\a": r"\a", "\b": r"\b", "\f": r"\f", "\n": r"\n", "\r": r"\r", "\t": r"\t", "\v": r"\v",
            "\\": r"\\", '"': r"\""}


def quote(s: str) -> str:
    """Go's strconv.Quote: printable characters as they are, the C escapes,
    other ASCII controls as \\xNN and other non-printable runes as \\uNNNN or
    \\UNNNNNNNN."""
    out = ['"']
    for ch in s:
        o = ord(ch)
        if ch in _ESCAPES:
            out.append(_ESCAPES[ch])
        elif o < 0x20 or o == 0x7F:
            out.append(f"\\x{o:02x}")
        elif o < 0x80 or (unicodedata.category(ch)[0] not in "CZ" or ch == " "):
            out.append(ch)
        elif o < 0x10000:
            out.append(f"\\u{o:04x}")
        else:
            out.append(f"\\U{o:08x}")
    out.append('"')
    return "".join(out)


def serialize(value: "Value", depth: int = 0) -> str:
    """octagon_emit.go:34-115 (serializeOctagonValueAtDepth)."""
    if isinstance(value, bool):
        return "true" if value else "false"
    if isinstance(value, int):
        return str(value)
    if isinstance(value, float):
        text = format_float_g(value)
        if not any(c in text for c in ".eE"):
            text += ".0"
        return text
    if isinstance(value, str):
        return quote(value)
    if isinstance(value, list):
        return "[" + ", ".join(serialize(v, depth) for v in value) + "]"
    if isinstance(value, Record):
        lines = []
        for name, v in value.fields:
            rendered = serialize(v, depth + 1)
            if isinstance(v, (int, float)) and not isinstance(v, bool):
                rendered = "(" + rendered + ")"
            lines.append(f"{'    ' * (depth + 1)}{name}: {rendered}")
        type_name = value.type_name.rsplit(".", 1)[-1]
        return f"{type_name} {{\n" + "\n".join(lines) + f"\n{'    ' * depth}}}"
    raise TypeError(f"value of type {type(value).__name__} is not representable in .octagon output")


def write(path: str, value: "Value", prefix: str = "") -> str:
    """octagon_emit.go:11-28 (WriteOctagon): the path must end in .octagon;
    a non-empty output prefix (output_path_prefix.go:31-41) is put before the
    file name as ``prefix.name``.  Returns the path written."""
    if not path.endswith(".octagon"):
        raise ValueError("WriteOctagon path must end with .octagon")
    if prefix:
        d, base = os.path.split(path)
        path = os.path.join(d, prefix + "." + base)
    with open(path, "w", encoding="utf-8") as f:
        f.write(serialize(value) + "\n")
    return path
