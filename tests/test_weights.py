"""The int32 .npy weight reader (artifacts.hpp:31-49, 86-92) on the host: shape,
ring words, the format errors of MappedWeights.  Runs without a GPU."""
import numpy as np
import pytest

import praghip
from praghip._lib import PraghipError


def _save(tmp_path, name, arr):
    p = tmp_path / name
    np.save(p, arr)
    return str(p)


def test_reads_shape_words_and_max(tmp_path):
    w = np.arange(-600, 600, dtype=np.int32).reshape(40, 30) * 1747
    w[0, 0] = -(1 << 20)
    w[1, 1] = (1 << 20)
    path = _save(tmp_path, "w.npy", w.astype("<i4"))
    with praghip.MappedWeights(path, 40, 30) as m:
        assert (m.rows, m.cols) == (40, 30)
        np.testing.assert_array_equal(m.array(), w)
        mask = (1 << 59) - 1
        for r, c in [(0, 0), (1, 1), (3, 7), (39, 29), (20, 15)]:
            assert m.at(r, c) == int(w[r, c]) & mask  # Python's & on a negative int sign-extends
        assert m.max_abs() == int(np.abs(w.astype(np.int64)).max())
        with pytest.raises(PraghipError, match="BAD_SHAPE"):
            m.at(40, 0)


def test_vector_and_version2(tmp_path):
    v = np.array([-3, 0, 7, -(1 << 31)], dtype="<i4")
    p = tmp_path / "v.npy"
    with open(p, "wb") as f:
        np.lib.format.write_array(f, v, version=(2, 0))
    with praghip.MappedWeights(str(p), 4, vector=True) as m:
        assert [m.at(i) for i in range(4)] == [int(x) & ((1 << 59) - 1) for x in v]


@pytest.mark.parametrize("case", ["shape", "dtype", "fortran", "truncated", "magic", "missing", "zero"])
def test_format_errors(tmp_path, case):
    w = np.ones((4, 6), dtype="<i4")
    rows, cols = 4, 6
    if case == "shape":
        path, rows = _save(tmp_path, "a.npy", w), 5
        code = "E_NPY_SHAPE"
    elif case == "dtype":
        path, code = _save(tmp_path, "a.npy", w.astype("<i8")), "E_NPY_FORMAT"
    elif case == "fortran":
        path, code = _save(tmp_path, "a.npy", np.asfortranarray(w)), "E_NPY_FORMAT"
    elif case == "truncated":
        path = _save(tmp_path, "a.npy", w)
        data = open(path, "rb").read()
        open(path, "wb").write(data[:-4])
        code = "E_NPY_SHAPE"
    elif case == "magic":
        path = str(tmp_path / "a.npy")
        open(path, "wb").write(b"NOTNUMPY" + bytes(200))
        code = "E_NPY_FORMAT"
    elif case == "missing":
        path, code = str(tmp_path / "none.npy"), "E_WEIGHT_FILE"
    else:
        path, rows, code = _save(tmp_path, "a.npy", w), 0, "BAD_SHAPE"
    with pytest.raises(PraghipError, match=code):
        praghip.MappedWeights(path, rows, cols)


def test_upload_split_rejects_out_of_range(tmp_path):
    """The host split of praghip_weights_upload_split refuses a weight outside
    the three-signed-byte range before any device call."""
    from praghip import _lib
    w = np.zeros((4, 8), dtype="<i4")
    w[2, 3] = 0x7F7F7F + 1
    with praghip.MappedWeights(_save(tmp_path, "big.npy", w), 4, 8) as m:
        rc = _lib.lib().praghip_weights_upload_split(m._handle(), 0, 1 << 20, None)
        assert rc == _lib.E_SHAPE and _lib.lib().praghip_last_error() == b"E_WEIGHT_RANGE"
