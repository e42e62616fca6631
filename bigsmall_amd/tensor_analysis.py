"""Routing of tensors before codec selection: the reference's
`tensor_analysis.analyze_tensors` (bigsmall/tensor_analysis.py:80-132).

Each tensor dict carries name, shape, dtype, item_bytes and raw (bytes). The
decision per tensor is one of:

  * "tied"      the tensor's bytes equal those of an earlier tensor with the
                same item size and shape (md5 of the raw bytes), and it has at
                least TIE_MIN_BYTES bytes (tensor_analysis.py:93-110). The dtype
                string is not part of the match, as in the reference;
  * "lowcard"   not tied, item size 1, 2 or 4, between 1 and MAX_LOWCARD_UNIQUE
                distinct element values, and at least LOWCARD_MIN_BYTES bytes
                (tensor_analysis.py:112-125);
  * "wpe_delta" not tied or lowcard: a 2-D tensor of at least WPE_MIN_ROWS rows,
                4 columns and WPE_MIN_TENSOR_BYTES bytes whose first 64 rows
                change little from row to row, measured on the integer bit
                patterns (tensor_analysis.py:54-73, 126-129);
  * "generic"   everything else.

The thresholds are the reference's (tensor_analysis.py:30-33). The encoder
(bigsmall_amd/encoder.py) turns the decisions into entries as the reference's
encoder does (encoder.py:381-396, 155-168): tied -> `tied_ref`, then fewer
than 512 bytes -> `raw`, then lowcard -> `special` (in containers written for
the reference's readers) and wpe_delta -> the generic selection, which is
what the reference's encoder falls back to when its blosc2 coder is missing.
"""
from __future__ import annotations

import hashlib

import numpy as np

MAX_LOWCARD_UNIQUE = 16           # at most this many distinct values
LOWCARD_MIN_BYTES = 256           # and at least this many bytes
TIE_MIN_BYTES = 1024              # tied only from this size on
WPE_DELTA_RATIO = 0.6             # row-to-row change at most this share of the spread
WPE_MIN_ROWS = 16
WPE_MIN_TENSOR_BYTES = 16 * 1024
_UNIQUE_SAMPLE = 4096             # elements looked at before the full count
_WPE_SAMPLE_ROWS = 64

_WORD = {1: "<u1", 2: "<u2", 4: "<u4"}


def _elements(raw, item_bytes: int) -> np.ndarray:
    return np.frombuffer(memoryview(raw).cast("B"), dtype=_WORD[item_bytes])


def distinct_values(raw, item_bytes: int, cap: int = MAX_LOWCARD_UNIQUE + 1) -> int:
    """The number of distinct element values, at most `cap`. A first sample of
    4096 elements with more than `cap` values ends the count early
    (tensor_analysis.py:37-51)."""
    a = _elements(raw, item_bytes)
    if a.size == 0:
        return 0
    head = a[:_UNIQUE_SAMPLE]
    if np.unique(head).size > cap:
        return cap
    return min(int(np.unique(a).size), cap)


def is_lowcard(raw, item_bytes: int) -> bool:
    if item_bytes not in _WORD:
        return False
    k = distinct_values(raw, item_bytes)
    return 0 < k <= MAX_LOWCARD_UNIQUE and len(raw) >= LOWCARD_MIN_BYTES


def is_wpe_candidate(raw, item_bytes: int, shape) -> bool:
    """Row-correlated 2-D tensor: over the first 64 rows, the standard
    deviation of the row-to-row differences of the bit patterns (as int64) is
    at most WPE_DELTA_RATIO times that of the patterns themselves, which must
    not be constant (tensor_analysis.py:54-73)."""
    if item_bytes not in _WORD or len(shape) != 2:
        return False
    rows, cols = int(shape[0]), int(shape[1])
    if rows < WPE_MIN_ROWS or cols < 4 or len(raw) < WPE_MIN_TENSOR_BYTES:
        return False
    top = _elements(raw, item_bytes)[: min(rows, _WPE_SAMPLE_ROWS) * cols].astype(np.int64).reshape(-1, cols)
    spread = float(top.std())
    if spread == 0.0:
        return False
    return float(np.diff(top, axis=0).std()) <= WPE_DELTA_RATIO * spread


def analyze_tensors(tensors: list[dict], md5s: list[str] | None = None) -> tuple[list[dict], dict[int, int]]:
    """(decisions, {follower index: master index}) with decisions[i] =
    {"kind": "lowcard" | "wpe_delta" | "tied" | "generic", "tied_to": index or
    None}, in the reference's shape (tensor_analysis.py:80-132). `md5s`, when
    given, are the hex md5s of the tensors' raw bytes (the encoder computes
    them for the header anyway)."""
    out = [{"kind": "generic", "tied_to": None} for _ in tensors]
    first_of: dict[tuple, int] = {}
    for i, t in enumerate(tensors):
        raw = t["raw"]
        if len(raw) < TIE_MIN_BYTES:
            continue
        key = (t["item_bytes"], tuple(t["shape"]), md5s[i] if md5s is not None else hashlib.md5(raw).hexdigest())
        master = first_of.setdefault(key, i)
        if master != i:
            out[i] = {"kind": "tied", "tied_to": master}
    for i, t in enumerate(tensors):
        if out[i]["kind"] != "generic" or t["item_bytes"] not in _WORD:
            continue
        if is_lowcard(t["raw"], t["item_bytes"]):
            out[i] = {"kind": "lowcard", "tied_to": None}
        elif is_wpe_candidate(t["raw"], t["item_bytes"], t["shape"]):
            out[i] = {"kind": "wpe_delta", "tied_to": None}
    return out, {i: d["tied_to"] for i, d in enumerate(out) if d["kind"] == "tied"}
