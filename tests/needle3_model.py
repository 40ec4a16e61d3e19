"""Needle 3 archives (needle_cs_amd/archive.py) and the oracle's engine over
them (oracle/needle3.py), under the names the tests use."""
from needle_cs_amd.archive import NEEDLE3, SMALL, hada_split, header_words, parse  # noqa: F401
from needle_cs_amd.archive import needle3_archive as write_archive  # noqa: F401
from oracle.needle3 import OracleEngine, OracleModel  # noqa: F401
