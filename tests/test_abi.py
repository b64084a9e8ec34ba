"""CPU checks of the drop-in boundary: the built library loads and exports
every function include/browservec_hip.h declares (no GPU calls)."""

import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "browservec_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\**\s*(bv_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_seam():
    names = declared_functions()
    for must in ("bv_device_open", "bv_index_create", "bv_index_append", "bv_index_query", "bv_index_query_masked",
                 "bv_index_query_batch", "bv_index_rerank", "bv_index_search", "bv_index_destroy", "bv_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from browservec_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libbrowservec_hip.so is not built (python -m browservec_amd.build)")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding covers the same set
    assert set(declared_functions()) <= set(_lib.SIGNATURES)


def test_no_device_error_path_is_clean():
    """Without a GPU, opening a device fails with a status code and message,
    never a crash or a silent CPU fallback."""
    from browservec_amd import _lib
    from browservec_amd.index import DeviceContext

    try:
        import torch

        if torch.cuda.is_available():
            pytest.skip("a GPU is present")
    except Exception:
        pass
    with pytest.raises(_lib.BVError) as e:
        DeviceContext(0)
    assert e.value.code in (_lib.BV_E_UNSUPPORTED, _lib.BV_E_HIP, _lib.BV_E_INVALID)


def test_struct_layouts_match_header():
    from browservec_amd import _lib

    import re
    from pathlib import Path

    header = (Path(__file__).resolve().parents[1] / "include" / "browservec_hip.h").read_text()
    for struct, cls in (("bv_index_desc", _lib.IndexDesc), ("bv_index_stats", _lib.IndexStats)):
        body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (struct, struct), header, re.S).group(1)
        body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
        fields = re.findall(r"(\w+)\s+(\w+);", body)
        assert [n for _, n in fields] == [n for n, _ in cls._fields_], struct
        ctype = {"uint32_t": ctypes.c_uint32, "uint64_t": ctypes.c_uint64, "float": ctypes.c_float,
                 "double": ctypes.c_double}
        assert [ctype[t] for t, _ in fields] == [t for _, t in cls._fields_], struct
    assert ctypes.sizeof(_lib.IndexDesc) == 19 * 4
    # IndexStats: u64 + 7*u32 + f32 + 3*f64 + 3*u64
    assert ctypes.sizeof(_lib.IndexStats) == 8 + 8 * 4 + 3 * 8 + 3 * 8


def test_query_lengths_are_checked_before_the_library():
    """The Python binding refuses a query whose length is not the index
    dimension (a short buffer would otherwise be read past its end); no
    device is needed because the check runs before any library call."""
    from browservec_amd import _lib as L
    from browservec_amd.index import IVFIndex, NativeIndex

    fake = NativeIndex.__new__(NativeIndex)
    fake.dim = 8
    fake.lib = None
    fake.handle = None
    for call in (lambda: fake.query(np.zeros(7, np.float32), 3),
                 lambda: fake.query_masked(np.zeros(9, np.float32), 3, np.ones(1, np.uint32)),
                 lambda: fake.query_batch(np.zeros(15, np.float32), 2, 3),
                 lambda: fake.search(np.zeros(12, np.float32), 4, 3),
                 lambda: fake.rerank(np.zeros(4, np.float32), [0, 1], 2)):
        with pytest.raises(L.BVError) as e:
            call()
        assert e.value.code == L.BV_E_INVALID and "floats, got" in str(e.value)
    fake_ivf = IVFIndex.__new__(IVFIndex)
    fake_ivf.dim = 8
    with pytest.raises(L.BVError):
        fake_ivf.export_probe_scores(np.zeros(12, np.float32))
