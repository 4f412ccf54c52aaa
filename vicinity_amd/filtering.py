"""Metadata filters for filtered IVF-PQ search (src/filtering/mod.rs:1-230).

A document's metadata is a dict from field name to a typed value: Int, Float,
Str or Bool (mod.rs:14-23).  Python values map onto them by type (bool before
int, since bool is an int in Python), and equality is typed: Int(2) is not
Float(2.0) (mod.rs:151-153 compares with the derived `PartialEq`).

IVFPQIndex.search_with_filter accepts only an equality on the index's filter
field with an integer category 0..63 (search.rs:1429-1457); the other
predicates exist so that callers meet the reference's errors and so that
`matches` can state the predicate semantics on the host.
"""

from __future__ import annotations

from dataclasses import dataclass
from dataclasses import field as dc_field
from typing import Any

_I64_MIN, _I64_MAX = -(1 << 63), (1 << 63) - 1


def metadata_value(v: Any) -> tuple[str, Any]:
    """The typed value (kind, value) of a Python value (mod.rs:14-23)."""
    if isinstance(v, bool):
        return ("bool", v)
    if isinstance(v, int):
        if not _I64_MIN <= v <= _I64_MAX:
            raise ValueError(f"integer metadata value {v} does not fit in 64 bits")
        return ("int", v)
    if isinstance(v, float):
        return ("float", v)
    if isinstance(v, str):
        return ("str", v)
    raise TypeError(f"unsupported metadata value type {type(v).__name__} "
                    "(use int, float, str or bool)")


def _partial_cmp(a: tuple[str, Any], b: tuple[str, Any]) -> int | None:
    """mod.rs:41-53: ordered within one kind only (NaN compares as unordered)."""
    if a[0] != b[0]:
        return None
    x, y = a[1], b[1]
    if x < y:
        return -1
    if x > y:
        return 1
    if x == y:
        return 0
    return None


@dataclass(frozen=True)
class MetadataFilter:
    """A metadata predicate (mod.rs MetadataFilter): equals, range, and, or."""

    kind: str
    field: str | None = None
    value: tuple[str, Any] | None = None
    min: tuple[str, Any] | None = None
    max: tuple[str, Any] | None = None
    predicates: tuple["MetadataFilter", ...] = dc_field(default_factory=tuple)

    @staticmethod
    def equals(field_name: str, value: Any) -> "MetadataFilter":
        return MetadataFilter("equals", field=field_name, value=metadata_value(value))

    @staticmethod
    def range(field_name: str, min: Any = None, max: Any = None) -> "MetadataFilter":
        return MetadataFilter("range", field=field_name,
                              min=None if min is None else metadata_value(min),
                              max=None if max is None else metadata_value(max))

    @staticmethod
    def and_(predicates) -> "MetadataFilter":
        return MetadataFilter("and", predicates=tuple(predicates))

    @staticmethod
    def or_(predicates) -> "MetadataFilter":
        return MetadataFilter("or", predicates=tuple(predicates))

    def matches(self, metadata: dict) -> bool:
        """mod.rs:151-174: whether a document's metadata satisfies the predicate."""
        if self.kind == "equals":
            if self.field not in metadata:
                return False
            v = metadata_value(metadata[self.field])
            return v[0] == self.value[0] and v[1] == self.value[1]
        if self.kind == "range":
            if self.field not in metadata:
                return False
            v = metadata_value(metadata[self.field])
            if self.min is not None:
                o = _partial_cmp(v, self.min)
                if o is None or o < 0:
                    return False
            if self.max is not None:
                o = _partial_cmp(v, self.max)
                if o is None or o > 0:
                    return False
            return True
        if self.kind == "and":
            return all(p.matches(metadata) for p in self.predicates)
        if self.kind == "or":
            return any(p.matches(metadata) for p in self.predicates)
        raise ValueError(f"unknown filter kind {self.kind!r}")


def filter_category(flt: MetadataFilter, filter_field: str | None) -> int:
    """The category an IVF-PQ filtered search looks for (search.rs:1429-1457),
    with the reference's errors: a predicate other than an equality is
    unsupported; the field must be the index's filter field; the value must be
    an integer in 0..63."""
    if not isinstance(flt, MetadataFilter):
        raise TypeError("filter must be a MetadataFilter")
    if flt.kind != "equals":
        raise ValueError("Unsupported: non-equality predicates on filter_field "
                         "(use only equality predicates on the configured filter_field)")
    if flt.field != filter_field:
        raise ValueError(f"filter field '{flt.field}' doesn't match index filter field "
                         f"'{filter_field!r}'")
    kind, v = flt.value
    if kind != "int":
        raise ValueError("category ID must be an integer in 0..63 for bitmask filtering")
    if not 0 <= v < 64:
        raise ValueError(f"category ID {v} exceeds bitmask limit of 63")
    return v


def metadata_category(metadata: dict, filter_field: str) -> int:
    """add_metadata's check of the filter field (search.rs:445-465): the
    category 0..63 it carries, or -1 when the metadata lacks the field."""
    if filter_field not in metadata:
        return -1
    kind, v = metadata_value(metadata[filter_field])
    if kind != "int":
        raise ValueError("category ID must be an integer in 0..63 for bitmask filtering")
    if not 0 <= v < 64:
        raise ValueError(f"category ID {v} exceeds bitmask limit of 63; use an integer in 0..63")
    return v
