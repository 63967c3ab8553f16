"""BLAS flag words and letters (`uplo`, `side`, `diag`, `trans*`).

Same accepted spellings and errors as trnblas/_flags.py:18-51 (drop-in): the
documented words and the BLAS letters, case-insensitive and stripped; any
other string raises ValueError. Transpose flags take bools (truth value) or
'N' / 'T'; 'C' is rejected (no conjugate transpose).
"""

from __future__ import annotations

_TABLES = {
    "uplo": {"upper": "upper", "u": "upper", "lower": "lower", "l": "lower"},
    "side": {"left": "left", "l": "left", "right": "right", "r": "right"},
    "diag": {
        "unit": "unit",
        "u": "unit",
        "nonunit": "nonunit",
        "non-unit": "nonunit",
        "n": "nonunit",
    },
}


def _word(kind: str, value) -> str:
    table = _TABLES[kind]
    if isinstance(value, str) and value.strip().lower() in table:
        return table[value.strip().lower()]
    choices = sorted(set(table.values()))
    raise ValueError(f"{kind} must be one of {choices} (or the BLAS letter); got {value!r}")


def uplo_flag(value) -> str:
    """'upper' or 'lower'."""
    return _word("uplo", value)


def side_flag(value) -> str:
    """'left' or 'right'."""
    return _word("side", value)


def diag_flag(value) -> str:
    """'unit' or 'nonunit'."""
    return _word("diag", value)


def trans_flag(value, name: str = "trans") -> bool:
    """A transpose flag as a bool: non-strings by truth value, 'N' / 'T'."""
    if isinstance(value, str):
        key = value.strip().lower()
        if key == "n":
            return False
        if key == "t":
            return True
        raise ValueError(f"{name} must be a bool or 'N' / 'T'; got {value!r}")
    return bool(value)
