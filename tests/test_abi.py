"""CPU checks of the C-ABI boundary: libneedle_hip.so loads, exports every
entry point include/needle_hip.h declares, and the ctypes struct mirrors have
the reference's C# sequential layouts.  No compute call (no GPU here)."""
import ctypes as C
import os
import re

import numpy as np

import needle_cs_amd as N

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "needle_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nhip_[a-z0-9_]+)\s*\(", text)))


def test_library_builds_in_tree_and_loads():
    assert os.path.exists(N.LIB_PATH), "run __graft_entry__.build() first"
    N.lib()


def test_every_declared_symbol_is_exported():
    names = declared_functions()
    assert len(names) >= 51
    handle = C.CDLL(N.LIB_PATH)
    missing = [n for n in names if not hasattr(handle, n)]
    assert not missing, missing
    # and every declaration has a ctypes prototype in the binding
    assert sorted(set(names) - set(N._PROTOS)) == []


def test_struct_layouts_match_reference():
    # src/Needle/Model.cs:36-42, Model.cs:8-34, Quant.cs:11-28, Blocks.cs:11-27
    assert C.sizeof(N.Codebook) == 100
    assert N.Codebook.byte_scale.offset == 96
    assert C.sizeof(N.Cq) == 40 and N.Cq.rows.offset == 24 and N.Cq.bits.offset == 32
    assert C.sizeof(N.Activations) == 40 and N.Activations.cols.offset == 24
    assert C.sizeof(N.AttnTile) == 128
    assert N.AttnTile.keys.offset == 24 and N.AttnTile.key_stride.offset == 56
    assert N.AttnTile.count.offset == 72 and N.AttnTile.scores.offset == 80
    assert N.AttnTile.probability_stride.offset == 104 and N.AttnTile.sums.offset == 120


def test_fill_kernel_table_argument_checks_without_gpu():
    table = (C.c_void_p * 27)()
    assert N.lib().nhip_fill_kernel_table(table, 27) == 0
    filled = [i for i in range(27) if table[i]]
    assert filled == [0, 1, 3, 4, 22]
    assert N.lib().nhip_fill_kernel_table(table, 26) != 0


def test_synthetic_generators_are_deterministic_and_match_oracle(orc):
    st1, st2 = C.c_uint64(0x5EED), orc.state(0x5EED)
    a = N.synth_int8(st1, 10000)
    b = orc.synth_int8(st2, 10000)
    assert np.array_equal(a, b) and a.min() >= -127 and a.max() <= 127
    st1, st2 = C.c_uint64(0x5EED), orc.state(0x5EED)
    x = N.synth_normal(st1, 20000)
    y = orc.synth_normal(st2, 20000)
    assert np.array_equal(x, y)
    assert abs(float(x.mean())) < 0.05 and abs(float(x.std()) - 1.0) < 0.05
    h = N.synth_half_uniform(C.c_uint64(3), 5000, 0.002, 0.02)
    hv = h.view(np.float16).astype(np.float32)
    assert hv.min() >= 0.002 - 1e-5 and hv.max() <= 0.02 + 1e-5
    assert np.array_equal(h, orc.synth_half_uniform(orc.state(3), 5000, 0.002, 0.02))
