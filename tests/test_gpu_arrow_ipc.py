"""Arrow IPC streams into and out of device relations (reference:
from_arrow_ipc_stream / to_arrow_ipc_stream / read_ / write_arrow_ipc_stream_file,
crates/xlog-cuda/src/provider/io.rs:697-773), checked against pyarrow and, end
to end, against the CPU oracle."""
import io
import sys

import numpy as np
import pyarrow as pa
import pyarrow.ipc as ipc
import pytest

import oracle
from xlog_amd import XlogError, datagen, tc_plan

pytestmark = pytest.mark.gpu


def _note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _stream(cols, names):
    rb = pa.record_batch([pa.array(c, pa.uint32()) for c in cols], names=names)
    sink = io.BytesIO()
    with ipc.new_stream(sink, rb.schema) as w:
        w.write_batch(rb)
    return sink.getvalue()


@pytest.mark.parametrize("arity", [1, 2, 3, 4])
@pytest.mark.parametrize("n", [0, 5, 1 << 20])
def test_ingest_packs_columns(provider, arity, n):
    _note(f"arrow ingest arity={arity} n={n}")
    p = provider
    rng = np.random.default_rng(arity * 31 + n)
    cols = [rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32) for _ in range(arity)]
    rel = p.from_arrow_ipc_stream(_stream(cols, [f"k{i}" for i in range(arity)]))
    assert rel.arity == arity and rel.num_rows() == n
    for i in range(arity):
        assert np.array_equal(p.download_column(rel, i), cols[i])
    # and back out: pyarrow reads what the device exported
    t = ipc.open_stream(p.to_arrow_ipc_stream(rel, names=[f"k{i}" for i in range(arity)])).read_all()
    assert t.schema.names == [f"k{i}" for i in range(arity)] and t.num_rows == n
    for i in range(arity):
        assert np.array_equal(t.column(i).to_numpy(), cols[i])


def test_file_forms_and_errors(provider, tmp_path):
    p = provider
    src, dst = datagen.random_digraph(500, 2000, 3)
    path = tmp_path / "edge.arrow"
    path.write_bytes(_stream([src, dst], ["src", "dst"]))
    e = p.read_arrow_ipc_stream_file(path)
    assert np.array_equal(p.download_column(e, 0), src) and np.array_equal(p.download_column(e, 1), dst)
    out = tmp_path / "copy.arrow"
    p.write_arrow_ipc_stream_file(e, out, names=["src", "dst"])
    t = ipc.open_stream(out.read_bytes()).read_all()
    assert np.array_equal(t.column("src").to_numpy(), src)
    with pytest.raises(XlogError) as ex:
        p.read_arrow_ipc_stream_file(tmp_path / "missing.arrow")
    assert ex.value.status == 1 and "Failed to read Arrow IPC stream from" in str(ex.value)
    bad = tmp_path / "bad.arrow"
    bad.write_bytes(b"\xff\xff\xff\xff\x10\x00\x00\x00" + b"\x00" * 4)
    with pytest.raises(XlogError):
        p.read_arrow_ipc_stream_file(bad)


def test_fixpoint_from_arrow_files(provider, tmp_path):
    """The CLI flow (--input edge=file.arrow, output written as Arrow): closure of an Arrow edge file,
    written back as Arrow, equal to the BFS closed form."""
    p = provider
    n = 1000
    src, dst = datagen.random_digraph(n, 5000, datagen.seed_for(1))
    path = tmp_path / "edge.arrow"
    path.write_bytes(_stream([src, dst], ["x", "y"]))
    outs, st = p.fixpoint(tc_plan(), [p.read_arrow_ipc_stream_file(path), None])
    res = tmp_path / "reach.arrow"
    p.write_arrow_ipc_stream_file(outs[1], res, names=["x", "y"])
    t = ipc.open_stream(res.read_bytes()).read_all()
    got = (t.column("x").to_numpy().astype(np.uint64) << np.uint64(32)) | t.column("y").to_numpy().astype(np.uint64)
    exp = oracle.bfs_tc(n, src, dst)
    assert np.array_equal(got, exp["relation"]) and st["iterations"] == exp["iterations"]
