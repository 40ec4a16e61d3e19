"""The .cact writer the reader's tests use (needle_cs_amd/archive.py)."""
from needle_cs_amd.archive import CQ, FP16, FP32, HEADER, MAGIC, RAW, RECORD, cq_payload, record_offsets, write  # noqa: F401
