"""Axis-family expansion: a textual rewrite applied before parsing.

Behaviour follows the reference (src/torch_einshard/families.py:5-128):

* ``*fam`` becomes the family's axes separated by spaces;
* ``[*a *b]`` becomes the zipped groups ``(a1 b1) (a2 b2) ...`` — unless the
  bracket content is an operand annotation (``[param, grad=...]``), which is left
  untouched;
* ``sizes`` / ``windows`` / ``radius`` / ``halos`` dictionaries keyed by a family
  name expand to one entry per member axis (a scalar value is repeated).

Expansion results are memoised (LRU, 1024 entries); callers receive copies.
"""

import re
from functools import lru_cache

__all__ = [
    "expand_axis_families",
    "cached_expand_axis_families",
    "expand_family_mapping",
]

_FAMILY_REF = re.compile(r"\*([A-Za-z0-9]+)")
_BRACKETS = re.compile(r"\[([^\]]+)\]")
_ANNOTATION_PREFIXES = ("param", "grad=", "init_sync=")


def _families_dict(families):
    if not families:
        return {}
    return {name: tuple(members) for name, members in families.items()}


def _hashable(mapping):
    if mapping is None or not isinstance(mapping, dict):
        return mapping
    items = []
    for key, value in mapping.items():
        items.append((key, tuple(value) if isinstance(value, (list, tuple)) else value))
    return ("__dict__", tuple(sorted(items)))


def _unhashable(key):
    if isinstance(key, tuple) and len(key) == 2 and key[0] == "__dict__":
        return dict(key[1])
    return key


def _member_name(axis_text: str) -> str:
    # a family member may carry a sharding suffix ("h/sp"); mappings key on the name
    return axis_text.split("/", 1)[0].strip()


def expand_family_mapping(mapping, families, *, label):
    """Expand dictionary keys that name a family into one key per member axis."""
    families = _families_dict(families)
    if not isinstance(mapping, dict) or not families:
        return mapping
    result = {}
    for key, value in mapping.items():
        if key not in families:
            result[key] = value
            continue
        members = families[key]
        if isinstance(value, (str, bytes)):
            values = (value,) * len(members)
        else:
            try:
                values = tuple(value)
            except TypeError:
                values = (value,) * len(members)
        if len(values) != len(members):
            raise ValueError(
                f"{label} family {key!r} has {len(values)} values for {len(members)} axes"
            )
        for member, member_value in zip(members, values):
            name = _member_name(member)
            if name in result and result[name] != member_value:
                raise ValueError(f"Conflicting {label.lower()} for expanded axis {name!r}")
            result[name] = member_value
    return result


def _looks_like_annotation(content: str) -> bool:
    parts = [re.sub(r"\s+", "", part) for part in content.split(",")]
    return all(any(part.startswith(prefix) for prefix in _ANNOTATION_PREFIXES) for part in parts)


def _zip_brackets(match, families):
    content = match.group(1)
    if _looks_like_annotation(content):
        return match.group(0)
    tokens = content.split()
    if not tokens or not all(token.startswith("*") for token in tokens):
        raise ValueError("Zipped axis-family groups must contain only family references")
    names = [token[1:] for token in tokens]
    for name in names:
        if name not in families:
            raise ValueError(f"Unknown axis family {name!r}")
    if len({len(families[name]) for name in names}) != 1:
        raise ValueError("Zipped axis families must have matching lengths")
    columns = zip(*(families[name] for name in names))
    return " ".join("(" + " ".join(column) + ")" for column in columns)


def expand_axis_families(expression, sizes=None, families=None):
    """Return ``(expanded_expression, expanded_sizes)``."""
    families = _families_dict(families)
    if not families:
        return expression, sizes

    def single(match):
        name = match.group(1)
        if name not in families:
            raise ValueError(f"Unknown axis family {name!r}")
        return " ".join(families[name])

    expression = _BRACKETS.sub(lambda match: _zip_brackets(match, families), expression)
    expression = _FAMILY_REF.sub(single, expression)
    return expression, expand_family_mapping(sizes, families, label="Size")


@lru_cache(maxsize=1024)
def _expand_cached(expression, sizes_key, families_key):
    return expand_axis_families(expression, _unhashable(sizes_key), dict(families_key))


def cached_expand_axis_families(expression, sizes=None, families=None):
    families_key = tuple(sorted(_families_dict(families).items()))
    expanded, expanded_sizes = _expand_cached(expression, _hashable(sizes), families_key)
    if isinstance(expanded_sizes, dict):
        expanded_sizes = dict(expanded_sizes)
    elif isinstance(expanded_sizes, list):
        expanded_sizes = list(expanded_sizes)
    return expanded, expanded_sizes
