"""Arrow IPC stream codec (xlog_amd/csrc/arrow_ipc.cpp) against pyarrow, the
independent implementation of the format: streams written here are read by
pyarrow, streams written by pyarrow are read here, and the error behaviour
follows the reference's from_arrow_ipc_stream (crates/xlog-cuda/src/provider/
io.rs:716-739).  Host only: no device is touched."""
import io

import numpy as np
import pyarrow as pa
import pyarrow.ipc as ipc
import pytest

from xlog_amd import XlogError, arrow_ipc_decode_u32, arrow_ipc_encode_u32

INVALID_ARG, TYPE_MISMATCH, UNSUPPORTED = 1, 2, 7


def _stream(batches, schema=None, options=None):
    sink = io.BytesIO()
    schema = schema if schema is not None else batches[0].schema
    with ipc.new_stream(sink, schema, options=options) as w:
        for b in batches:
            w.write_batch(b)
    return sink.getvalue()


def _cols(n, arity, seed):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32) for _ in range(arity)]


@pytest.mark.parametrize("arity", [1, 2, 3, 4])
@pytest.mark.parametrize("n", [0, 1, 7, 1000])
def test_encode_is_read_by_pyarrow(arity, n):
    cols = _cols(n, arity, 10 * arity + n)
    data = arrow_ipc_encode_u32(cols)
    t = ipc.open_stream(data).read_all()
    assert t.num_rows == n and t.num_columns == arity
    assert t.schema.names == [f"c{i}" for i in range(arity)]
    for i in range(arity):
        assert t.schema.field(i).type == pa.uint32() and not t.schema.field(i).nullable
        assert np.array_equal(t.column(i).to_numpy(), cols[i])
    # and decodes back here
    back = arrow_ipc_decode_u32(data)
    assert len(back) == arity and all(np.array_equal(a, b) for a, b in zip(back, cols))


def test_encode_names():
    data = arrow_ipc_encode_u32(_cols(5, 2, 1), names=["src", "dst"])
    assert ipc.open_stream(data).read_all().schema.names == ["src", "dst"]
    with pytest.raises(XlogError):
        arrow_ipc_encode_u32(_cols(5, 2, 1), names=["only_one"])


@pytest.mark.parametrize("arity", [1, 2, 4])
@pytest.mark.parametrize("n", [0, 3, 4097])
def test_pyarrow_stream_is_decoded(arity, n):
    cols = _cols(n, arity, 7 + n)
    rb = pa.record_batch([pa.array(c, pa.uint32()) for c in cols], names=[f"col{i}" for i in range(arity)])
    back = arrow_ipc_decode_u32(_stream([rb]))
    assert len(back) == arity and all(np.array_equal(a, b) for a, b in zip(back, cols))


@pytest.mark.parametrize("opts", [ipc.IpcWriteOptions(metadata_version=ipc.MetadataVersion.V4),
                                  ipc.IpcWriteOptions(use_legacy_format=True)],
                         ids=["metadata-v4", "legacy-no-continuation"])
def test_older_stream_forms(opts):
    cols = _cols(100, 2, 3)
    rb = pa.record_batch([pa.array(c, pa.uint32()) for c in cols], names=["a", "b"])
    back = arrow_ipc_decode_u32(_stream([rb], options=opts))
    assert all(np.array_equal(a, b) for a, b in zip(back, cols))


def test_sliced_batch():
    cols = _cols(300, 2, 4)
    rb = pa.record_batch([pa.array(c, pa.uint32()) for c in cols], names=["a", "b"]).slice(17, 200)
    back = arrow_ipc_decode_u32(_stream([rb]))
    assert all(np.array_equal(a, b[17:217]) for a, b in zip(back, cols))


def test_nulls_take_stored_values():
    """io.rs:651-653 reads values() and ignores validity: null slots keep the stored value."""
    arr = pa.array([5, None, 7, None], pa.uint32())
    rb = pa.record_batch([arr], names=["a"])
    stored = np.frombuffer(arr.buffers()[1], dtype=np.uint32)[:4]
    back = arrow_ipc_decode_u32(_stream([rb]))
    assert np.array_equal(back[0], stored) and back[0][0] == 5 and back[0][2] == 7


def test_batch_count_errors_match_reference():
    rb = pa.record_batch([pa.array([1, 2], pa.uint32())], names=["a"])
    with pytest.raises(XlogError) as ex:
        arrow_ipc_decode_u32(_stream([rb, rb]))
    assert ex.value.status == INVALID_ARG and "multiple record batches" in str(ex.value)
    with pytest.raises(XlogError) as ex:
        arrow_ipc_decode_u32(_stream([], schema=rb.schema))
    assert ex.value.status == INVALID_ARG and "no record batches" in str(ex.value)


@pytest.mark.parametrize("typ", [pa.int32(), pa.uint64(), pa.int64(), pa.float32(), pa.uint16(), pa.bool_()])
def test_other_column_types_refused(typ):
    rb = pa.record_batch([pa.array([1, 0, 1], pa.int64()).cast(typ)], names=["a"])
    with pytest.raises(XlogError) as ex:
        arrow_ipc_decode_u32(_stream([rb]))
    assert ex.value.status == TYPE_MISMATCH


def test_compression_and_dictionaries_refused():
    rb = pa.record_batch([pa.array(np.arange(1000, dtype=np.uint32))], names=["a"])
    for codec in ("lz4", "zstd"):
        if pa.Codec.is_available(codec):
            with pytest.raises(XlogError) as ex:
                arrow_ipc_decode_u32(_stream([rb], options=ipc.IpcWriteOptions(compression=codec)))
            assert ex.value.status == UNSUPPORTED
    d = pa.array([1, 2, 1], pa.uint32()).dictionary_encode()
    with pytest.raises(XlogError) as ex:
        arrow_ipc_decode_u32(_stream([pa.record_batch([d], names=["a"])]))
    assert ex.value.status in (TYPE_MISMATCH, UNSUPPORTED)


def test_arity_limits():
    rb = pa.record_batch([pa.array([1], pa.uint32()) for _ in range(5)], names=list("abcde"))
    with pytest.raises(XlogError) as ex:
        arrow_ipc_decode_u32(_stream([rb]))
    assert ex.value.status == UNSUPPORTED
    with pytest.raises(XlogError):
        arrow_ipc_encode_u32([])


def test_malformed_streams_never_crash():
    """Every truncation and a sample of bit flips of a valid stream either decodes or is INVALID_ARG-class
    (no out-of-bounds read: every metadata access is bounds-checked)."""
    cols = _cols(50, 2, 5)
    good = arrow_ipc_encode_u32(cols)
    for cut in range(len(good)):
        try:
            arrow_ipc_decode_u32(good[:cut])
        except XlogError as e:
            assert e.status in (INVALID_ARG, TYPE_MISMATCH, UNSUPPORTED)
    rng = np.random.default_rng(6)
    for _ in range(3000):
        b = bytearray(good)
        pos = int(rng.integers(0, len(b)))
        b[pos] ^= 1 << int(rng.integers(0, 8))
        try:
            out = arrow_ipc_decode_u32(bytes(b))
            assert 1 <= len(out) <= 4
        except XlogError as e:
            assert e.status in (INVALID_ARG, TYPE_MISMATCH, UNSUPPORTED)
    for junk in (b"", b"\x00" * 8, b"\xff" * 16, bytes(range(64))):
        with pytest.raises(XlogError):
            arrow_ipc_decode_u32(junk)
