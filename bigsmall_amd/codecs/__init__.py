"""Codec plugins of the decode engine (shape of bigsmall/codecs)."""
