"""ORACLE — test infrastructure, not part of the product.

CPU restatement (plain C, oracle/bs_oracle.c) of the reference BigSmall
rANS-family codecs. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline legs may import this package: to check results against, as the
timed CPU baseline, and to write the reference-format blobs that baseline
decodes; the product package bigsmall_amd never imports it.
"""
from .oracle import *  # noqa: F401,F403
