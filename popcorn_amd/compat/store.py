"""Record persistence: bundled reports plus the per-user cache, newest conclusive row winning.

Behaviour follows bench/store.py:
  * the user cache is `$POPCORN_CACHE_DIR` (else `$XDG_CACHE_HOME/popcorn`,
    else `~/.cache/popcorn`) + `/v3/reports/<op>.jsonl` (:62-72);
  * bundled rows live in `<op>.parquet` or `<op>.jsonl` of a reports
    directory (:149-153); Parquet files have the stated 21-column schema, with
    config/fwd/bwd/bench as JSON text (sorted keys) and zstd compression
    (:31-57, 116-133), so files written here and Popcorn's load in either;
  * `read(directory)` returns every row of a reports directory (:148-151),
    `scrub` rewrites it without selected rows (:382-409), and `publish` upserts
    the user cache's rows into `<op>.parquet` files, the offline half of
    Popcorn's publish step (bench/__main__.py:305-308);
  * `write` upserts by `Record.key` under a process lock plus `flock`, via a
    temporary file and `os.replace` (:102-113, 358-379);
  * `merged(op)` overlays bundled and user rows by key minus the op name,
    preferring conclusive rows, then newer timestamps, then the user cache
    (:96-99, 442-451).
"""

from __future__ import annotations

import json
import os
from collections import defaultdict
from collections.abc import Iterable, Iterator, Mapping
from contextlib import contextmanager
from pathlib import Path
from threading import Lock
from typing import Any

from popcorn_amd.compat.records import SCHEMA, Call, Record

try:
    import fcntl
except ImportError:  # pragma: no cover - non-POSIX
    fcntl = None

BUNDLED_REPORTS = Path(__file__).resolve().parent / "reports"
PUBLISHED = ".parquet"
SCRATCH = ".jsonl"
NESTED = ("config", "fwd", "bwd", "bench")
_LOCK = Lock()


def user_reports() -> Path:
    root = os.getenv("POPCORN_CACHE_DIR")
    if root is None:
        root = str(Path(os.getenv("XDG_CACHE_HOME", str(Path.home() / ".cache"))) / "popcorn")
    return Path(root).expanduser() / f"v{SCHEMA}" / "reports"


def conclusive(record: Record) -> bool:
    return record.result.status in ("pass", "fail", "crash", "oom")


def unmeasured(record: Record | None, benchmark: bool = True) -> bool:
    """Should a run still produce this row: absent, inconclusive, or (for a benchmark) untimed?"""
    if record is None:
        return True
    status = record.result.status
    if benchmark and status == "pass" and not record.result.benchmarked:
        return True
    return status not in ("pass", "fail", "crash")


def matching(expected: str | None, recorded: str | None) -> bool:
    """Fingerprints agree; code that cannot be hashed (None) accepts any row."""
    return expected is None or expected == recorded


def prefer(record: Record, current: Record, priority: int = 0, current_priority: int = 0) -> bool:
    return (conclusive(record), record.environment.ts, priority) >= (
        conclusive(current), current.environment.ts, current_priority)


@contextmanager
def _locked(path: Path) -> Iterator[None]:
    with _LOCK:
        with path.with_suffix(path.suffix + ".lock").open("a") as handle:
            if fcntl is not None:
                fcntl.flock(handle, fcntl.LOCK_EX)
            try:
                yield
            finally:
                if fcntl is not None:
                    fcntl.flock(handle, fcntl.LOCK_UN)


def _parquet_schema():
    import pyarrow as pa

    columns = {
        "schema": pa.int32(), "op": pa.string(), "impl": pa.string(), "case": pa.string(), "case_id": pa.string(),
        "device": pa.string(), "torch": pa.string(), "backend_version": pa.string(), "ts": pa.string(),
        "ref_hash": pa.string(), "impl_hash": pa.string(), "status": pa.string(), "reason": pa.string(),
        "grad": pa.bool_(), "benchmarked": pa.bool_(), "bench_error": pa.string(), "reps": pa.int32(),
    }
    columns.update({name: pa.string() for name in NESTED})
    return pa.schema(columns)


def read_parquet(path: Path) -> list[Record]:
    import pyarrow.parquet as pq

    rows = pq.read_table(path).to_pylist()
    for row in rows:
        for name in NESTED:
            row[name] = json.loads(row[name]) if row.get(name) else {}
    return [Record.from_dict(row) for row in rows]


def write_parquet(records: Iterable[Record], path: Path) -> None:
    import pyarrow as pa
    import pyarrow.parquet as pq

    rows = []
    for record in records:
        row = record.to_dict()
        for name in NESTED:
            row[name] = json.dumps(row.get(name) or {}, sort_keys=True)
        rows.append(row)
    pq.write_table(pa.Table.from_pylist(rows, schema=_parquet_schema()), path, compression="zstd")


def read_file(path: Path | str) -> list[Record]:
    path = Path(path)
    try:
        if path.suffix == PUBLISHED:
            return read_parquet(path)
        return [Record.from_dict(json.loads(line)) for line in path.read_text().splitlines() if line.strip()]
    except FileNotFoundError:
        return []


def read(directory: Path | str) -> list[Record]:
    """Every row of a reports directory: its Parquet files, then its JSONL files, each in name order."""
    directory = Path(directory)
    paths = sorted(directory.glob(f"*{PUBLISHED}")) + sorted(directory.glob(f"*{SCRATCH}"))
    return [record for path in paths for record in read_file(path)]


def bundled_path(directory: Path, op: str) -> Path:
    published = directory / f"{op}{PUBLISHED}"
    return published if published.exists() else directory / f"{op}{SCRATCH}"


def _dump(records: list[Record], path: Path, suffix: str) -> None:
    if suffix == PUBLISHED:
        write_parquet(records, path)
    else:
        path.write_text("".join(json.dumps(r.to_dict(), sort_keys=True) + "\n" for r in records))


def write(records: Iterable[Record], directory: Path | str, suffix: str = SCRATCH) -> None:
    """Upsert rows into `<directory>/<op><suffix>`, one file per op, atomically."""
    directory = Path(directory)
    directory.mkdir(parents=True, exist_ok=True)
    by_op: dict[str, list[Record]] = defaultdict(list)
    for record in records:
        by_op[record.op].append(record)
    for op, incoming in sorted(by_op.items()):
        path = directory / f"{op}{suffix}"
        with _locked(path):
            rows = {r.key: r for r in read_file(path)}
            for record in incoming:
                if record.key not in rows or prefer(record, rows[record.key]):
                    rows[record.key] = record
            order = sorted(rows, key=lambda key: tuple("" if v is None else str(v) for v in key))
            tmp = path.with_name(f".{path.name}.{os.getpid()}.tmp")
            try:
                _dump([rows[k] for k in order], tmp, suffix)
                os.replace(tmp, path)
            finally:
                tmp.unlink(missing_ok=True)


def scrub(directory: Path | str, drop) -> int:
    """Rewrite a reports directory without the rows `drop(record)` selects; files left empty are
    removed. Returns the number of rows dropped."""
    directory = Path(directory)
    dropped = 0
    for path in sorted(directory.glob(f"*{PUBLISHED}")) + sorted(directory.glob(f"*{SCRATCH}")):
        with _locked(path):
            rows = read_file(path)
            kept = [r for r in rows if not drop(r)]
            if len(kept) == len(rows):
                continue
            dropped += len(rows) - len(kept)
            if not kept:
                path.unlink()
                continue
            tmp = path.with_name(f".{path.name}.{os.getpid()}.tmp")
            try:
                _dump(kept, tmp, path.suffix)
                os.replace(tmp, path)
            finally:
                tmp.unlink(missing_ok=True)
    return dropped


def publish(directory: Path | str, ops: Iterable[str] | None = None, user: Path | str | None = None) -> int:
    """Upsert the user cache's rows (all ops, or those named) into `<directory>/<op>.parquet`.

    The result is a reports directory in Popcorn's published format: rows from
    this device merge into it by key exactly as Popcorn's own writes do.
    Returns the number of rows offered.
    """
    source = Path(user) if user is not None else user_reports()
    wanted = None if ops is None else set(ops)
    rows = [r for path in sorted(source.glob(f"*{SCRATCH}")) for r in read_file(path)
            if wanted is None or r.op in wanted]
    write(rows, directory, PUBLISHED)
    return len(rows)


class Store:
    """Merged view over a bundled reports directory and the user cache."""

    def __init__(self, bundled: Path | str | None = None, user: Path | str | None = None) -> None:
        self._bundled = Path(bundled) if bundled is not None else None
        self._user = Path(user) if user is not None else None

    @property
    def bundled(self) -> Path:
        # read at use time so tests (and callers) can repoint the module default
        return self._bundled if self._bundled is not None else BUNDLED_REPORTS

    @property
    def user(self) -> Path:
        return self._user if self._user is not None else user_reports()

    def merged(self, op: str) -> tuple[Record, ...]:
        best: dict[tuple, tuple[int, Record]] = {}
        paths = list(dict.fromkeys((bundled_path(self.bundled, op), self.user / f"{op}{SCRATCH}")))
        for priority, path in enumerate(paths):
            for record in read_file(path):
                key = record.key[1:]
                if key not in best or prefer(record, best[key][1], priority, best[key][0]):
                    best[key] = (priority, record)
        return tuple(record for _, record in best.values())

    def exact(
        self, op: str, impl: str, call: Call, torch_version: str, backend_version: str | None,
        records: Iterable[Record] | None = None, ref_hash: str | None = None, impl_hash: str | None = None,
    ) -> Record | None:
        rows = self.merged(op) if records is None else records
        found = [
            r for r in rows
            if r.impl == impl
            and r.environment.device == call.device_name
            and r.environment.torch == torch_version
            and r.environment.backend_version == backend_version
            and r.result.grad == call.grad
            and r.config == call.config
            and matching(ref_hash, r.environment.ref_hash)
            and matching(impl_hash, r.environment.impl_hash)
        ]
        return max(found, key=lambda r: (conclusive(r), r.environment.ts), default=None)

    def reference_bench(
        self, op: str, case_id: str, config: Mapping[str, Any], device: str, torch_version: str, grad: bool,
        ref_hash: str | None,
    ) -> dict[str, float] | None:
        """Reusable torch timings of this exact case (never correctness evidence)."""
        found = [
            r for r in self.merged(op)
            if r.impl == "torch" and r.case_id == case_id and r.config == config
            and r.environment.device == device and r.environment.torch == torch_version
            and r.environment.backend_version is None and r.result.grad == grad
            and r.result.status == "pass" and r.result.benchmarked
            and matching(ref_hash, r.environment.ref_hash)
        ]
        latest = max(found, key=lambda r: r.environment.ts, default=None)
        if latest is None:
            return None
        bench = {k: v for k, v in latest.result.bench.items() if k.startswith("ref_")}
        bench.update({f"ref_{k}": v for k, v in latest.result.bench.items() if k.startswith(("fwd_", "bwd_"))})
        return bench if "ref_fwd_ms" in bench else None

    def write_user(self, records: Iterable[Record]) -> None:
        write(records, self.user)

    def write_bundled(self, records: Iterable[Record]) -> None:
        write(records, self.bundled, PUBLISHED)
