""".npy I/O of libcppnet (Utils::save_npy / load_npy_*, host-only, no GPU).

Pinned against numpy's own reader and writer, which fix the format
independently: a file we write must np.load to the logical tensor (our data
is ColMajor, so the header must say fortran_order True), and files numpy
writes in either order must read back as that tensor's ColMajor data.  The
header layout is the reference's (tensor_io.cpp:29-58): version 1.0, the dict
text, space padding before the newline so the data starts at a multiple of 64.
"""
import numpy as np
import pytest

from cppnet_amd import trainer

SHAPES = [(7,), (3, 5), (2, 3, 4), (2, 1, 3, 5), (1, 1), (4, 0)]


def _logical(rng, shape):
    return rng.standard_normal(shape).astype(np.float32)


@pytest.mark.parametrize("shape", SHAPES)
def test_write_is_numpy_readable(tmp_path, shape):
    a = _logical(np.random.default_rng(len(shape)), shape)
    path = tmp_path / "a.npy"
    trainer.npy_save(path, a.ravel(order="F"), list(shape))
    b = np.load(path)
    assert b.dtype == np.float32 and b.shape == shape
    np.testing.assert_array_equal(b, a)
    raw = path.read_bytes()
    assert raw[:8] == b"\x93NUMPY\x01\x00"
    hlen = int.from_bytes(raw[8:10], "little")
    assert (10 + hlen) % 64 == 0 and raw[10 + hlen - 1:10 + hlen] == b"\n"
    header = raw[10:10 + hlen].decode("latin1")
    assert header.startswith("{'descr': '<f4', 'fortran_order': True, 'shape': (")
    assert len(raw) == 10 + hlen + 4 * a.size


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("order", ["C", "F"])
def test_read_numpy_files(tmp_path, shape, order):
    a = _logical(np.random.default_rng(11), shape)
    path = tmp_path / "a.npy"
    np.save(path, np.asarray(a, order=order))
    data, dims = trainer.npy_load(path)
    assert dims == list(shape)
    np.testing.assert_array_equal(data, a.ravel(order="F"))


def test_raw_colmajor_reads_reference_files(tmp_path):
    """A file as the reference writes it: ColMajor bytes under fortran_order
    False (tensor_io.cpp:33).  raw_colmajor takes the bytes as they are, which
    is what the reference's reader does; the default follows the flag."""
    a = _logical(np.random.default_rng(5), (3, 4))
    d = "{'descr': '<f4', 'fortran_order': False, 'shape': (3, 4), }\n"
    pad = (64 - (10 + len(d)) % 64) % 64
    d = d[:-1] + " " * pad + "\n"
    path = tmp_path / "ref.npy"
    path.write_bytes(b"\x93NUMPY\x01\x00" + len(d).to_bytes(2, "little") + d.encode()
                     + a.ravel(order="F").tobytes())
    raw, dims = trainer.npy_load(path, raw_colmajor=True)
    assert dims == [3, 4]
    np.testing.assert_array_equal(raw, a.ravel(order="F"))
    flagged, _ = trainer.npy_load(path)
    # honouring the flag reads the bytes as C order: numpy's view of the file
    np.testing.assert_array_equal(flagged, np.load(path).ravel(order="F"))


def test_read_errors(tmp_path):
    bad = tmp_path / "bad.npy"
    bad.write_bytes(b"NOTNPY" + b"\x00" * 64)
    with pytest.raises(Exception, match="bad magic"):
        trainer.npy_load(bad)
    f64 = tmp_path / "f64.npy"
    np.save(f64, np.zeros((2, 2)))
    with pytest.raises(Exception, match="float32"):
        trainer.npy_load(f64)
    with pytest.raises(Exception, match="rank"):
        trainer.npy_save(tmp_path / "x.npy", np.zeros(1, np.float32), [])
