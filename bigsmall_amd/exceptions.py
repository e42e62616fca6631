"""Public exception types (mirrors bigsmall/exceptions.py:16-27)."""
from __future__ import annotations


class BigSmallVersionError(Exception):
    """A .bs container or codec needs a decoder this engine does not have.

    Same constructor and message shape as the reference's
    BigSmallVersionError (bigsmall/exceptions.py:16-27).
    """

    def __init__(self, required: str, installed: str, *, detail: str | None = None):
        self.required = required
        self.installed = installed
        msg = (f"This file requires bigsmall >= {required} (you have {installed}).\n"
               "Run: pip install --upgrade bigsmall")
        if detail:
            msg += f"\n({detail})"
        super().__init__(msg)


class DecodeError(ValueError):
    """A blob failed a device-side integrity check (bad header, bounds, or a
    rANS stream that did not end in the encoder's start state)."""
