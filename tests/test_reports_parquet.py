"""Schema-3 report files: Popcorn's published Parquet layout, read and written here.

The column spec below restates bench/store.py:31-57 (names, order, types) and
the nested-column rule of :116-133 (JSON text with sorted keys, zstd); the
round-trip, typed-null and Parquet-over-JSONL cases follow the reference's
own tests (tests/core/test_bench.py:498-528).
"""

from __future__ import annotations

import json

import pyarrow as pa
import pyarrow.parquet as pq
import pytest
import torch

from popcorn_amd.compat import store
from popcorn_amd.compat.records import Environment, Gauge, Record, Result

POPCORN_COLUMNS = [
    ("schema", pa.int32()), ("op", pa.string()), ("impl", pa.string()), ("case", pa.string()),
    ("case_id", pa.string()), ("device", pa.string()), ("torch", pa.string()), ("backend_version", pa.string()),
    ("ts", pa.string()), ("ref_hash", pa.string()), ("impl_hash", pa.string()), ("status", pa.string()),
    ("reason", pa.string()), ("grad", pa.bool_()), ("benchmarked", pa.bool_()), ("bench_error", pa.string()),
    ("reps", pa.int32()), ("config", pa.string()), ("fwd", pa.string()), ("bwd", pa.string()), ("bench", pa.string()),
]


def _record(status="pass", case_id="case", ts="2026-01-01T00:00:00+00:00", impl="fast", backend_version=None):
    result = Result(status=status, grad=True, fwd={"out0": Gauge(1e-3, 2e-3, 3.0)}, bwd={"x": Gauge(4e-3, 5e-3, 1.0)},
                    bench={"fwd_ms": 0.5, "ref_fwd_ms": 2.0}, benchmarked=True, reps=10)
    env = Environment("AMD Instinct MI355X", torch.__version__, backend_version, ts, "r0", "i0")
    config = {"dims": {"D": 4}, "batch": [2], "dtype": "bfloat16", "args": {"eps": 1e-6}, "present": []}
    return Record("op", impl, "D=4,batch=(2,),bfloat16,eps=1e-06", case_id, config, env, result)


def test_written_file_has_popcorns_columns_types_and_codec(tmp_path):
    store.write([_record(), _record("fail", "other", backend_version="0.1.0")], tmp_path, store.PUBLISHED)
    path = tmp_path / "op.parquet"
    schema = pq.read_schema(path)
    assert [(f.name, f.type) for f in schema] == POPCORN_COLUMNS
    meta = pq.ParquetFile(path).metadata
    for g in range(meta.num_row_groups):
        for c in range(meta.num_columns):
            assert meta.row_group(g).column(c).compression == "ZSTD"
    rows = pq.read_table(path).to_pylist()
    for row, record in zip(rows, sorted([_record(), _record("fail", "other", backend_version="0.1.0")],
                                        key=lambda r: tuple("" if v is None else str(v) for v in r.key))):
        for name in store.NESTED:
            assert row[name] == json.dumps(record.to_dict()[name], sort_keys=True)


def test_reads_a_file_laid_out_by_popcorns_writer(tmp_path):
    """A file built column by column to the spec (as bench/store.py:125-133 does) loads into equal records."""
    records = [_record(), _record("crash", "c2", impl="mi355x", backend_version="0.1.0")]
    rows = []
    for r in records:
        row = r.to_dict()
        for name in store.NESTED:
            row[name] = json.dumps(row[name], sort_keys=True)
        rows.append(row)
    pq.write_table(pa.Table.from_pylist(rows, schema=pa.schema(POPCORN_COLUMNS)), tmp_path / "op.parquet",
                   compression="zstd")
    back = store.read_file(tmp_path / "op.parquet")
    assert [r.to_dict() for r in back] == [r.to_dict() for r in records]


def test_published_rows_round_trip_and_typed_null_columns(tmp_path):
    records = [_record(), _record("fail", "other")]
    store.write(records, tmp_path, store.PUBLISHED)
    assert [r.to_dict() for r in store.read(tmp_path)] == [r.to_dict() for r in records]
    assert store.read(tmp_path)[0].environment.backend_version is None
    assert pq.read_schema(tmp_path / "op.parquet").field("backend_version").type == pa.string()


def test_published_parquet_is_preferred_over_scratch_jsonl(tmp_path):
    store.write([_record("fail")], tmp_path, store.PUBLISHED)
    store.write([_record("pass")], tmp_path)
    assert store.bundled_path(tmp_path, "op").suffix == store.PUBLISHED
    assert store.read_file(store.bundled_path(tmp_path, "op"))[0].result.status == "fail"
    assert len(store.read(tmp_path)) == 2  # Parquet rows, then JSONL rows


def test_publish_upserts_the_user_cache_into_parquet(tmp_path):
    user, reports = tmp_path / "cache", tmp_path / "reports"
    store.write([_record("pass", "a", ts="2026-02-01T00:00:00+00:00", impl="mi355x", backend_version="0.1.0"),
                 _record("pass", "b", impl="mi355x", backend_version="0.1.0")], user)
    other = _record("pass", "z")
    other.op = "other_op"
    store.write([other], user)
    store.write([_record("fail", "a", ts="2026-01-01T00:00:00+00:00", impl="mi355x", backend_version="0.1.0")],
                reports, store.PUBLISHED)
    assert store.publish(reports, ops=["op"], user=user) == 2
    rows = {r.case_id: r for r in store.read_file(reports / "op.parquet")}
    assert set(rows) == {"a", "b"} and rows["a"].result.status == "pass"  # newer conclusive row replaces
    assert not (reports / "other_op.parquet").exists()
    merged = store.Reports(bundled=reports, user=tmp_path / "empty").rows("op")
    assert sorted(r.case_id for r in merged) == ["a", "b"]


def test_scrub_drops_rows_and_removes_emptied_files(tmp_path):
    store.write([_record("error", "x"), _record("pass", "y")], tmp_path, store.PUBLISHED)
    lone = _record("error", "w")
    lone.op = "lone"
    store.write([lone], tmp_path)
    assert store.scrub(tmp_path, lambda r: r.result.status == "error") == 2
    assert [r.case_id for r in store.read(tmp_path)] == ["y"]
    assert not (tmp_path / "lone.jsonl").exists()


def test_rows_of_another_schema_are_refused(tmp_path):
    row = _record().to_dict()
    row["schema"] = 2
    (tmp_path / "op.jsonl").write_text(json.dumps(row) + "\n")
    with pytest.raises(ValueError, match="schema"):
        store.read_file(tmp_path / "op.jsonl")
