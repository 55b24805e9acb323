"""Report files: schema-3 rows on disk, and the merged view dispatch reads.

Rows live in two formats, one file per op:

  * JSONL (`<op>.jsonl`): the per-user cache that `op.benchmark(...)` and
    lazy bench mode append to, under `$POPCORN_CACHE_DIR/v3/reports/`
    (`~/.cache/popcorn/v3/reports/` by default);
  * Parquet (`<op>.parquet`): Popcorn's published layout -- the 21 typed
    columns of `COLUMNS` in that order, the nested fields (`config`, `fwd`,
    `bwd`, `bench`) as JSON text with sorted keys, zstd compression
    (bench/store.py:31-57, 116-133). Files written here load in Popcorn and
    the other way round.

A row's identity is `Record.key` (op, impl, device, case, grad, torch
version, backend version). When two rows share it, the one that ranks higher
by (conclusive, timestamp, source priority) is kept: a conclusive outcome
(pass / fail / crash / oom) outranks an inconclusive one (error / skip)
whatever their ages, so a flaky harness run cannot erase a known failure, and
between equals the newer row wins. Writes replace whole files atomically
under a process lock plus an advisory file lock, so concurrent writers
(threads or processes) never interleave rows.
"""

from __future__ import annotations

import json
import os
import threading
from collections import defaultdict
from collections.abc import Callable, Iterable, Iterator
from contextlib import contextmanager
from pathlib import Path
from typing import Any

import pyarrow as pa
import pyarrow.parquet as pq

from popcorn_amd.compat.records import SCHEMA, Record

try:
    import fcntl
except ImportError:  # pragma: no cover - every supported platform has it
    fcntl = None

# Published reports shipped beside the package; Popcorn fetches its own from the
# Hugging Face dataset, which is not reachable here, so this stays empty unless
# rows are published into it.
BUNDLED_REPORTS = Path(__file__).resolve().parent / "reports"
PUBLISHED = ".parquet"
SCRATCH = ".jsonl"

# Popcorn's published column layout: names, order and types are a format.
NESTED = ("config", "fwd", "bwd", "bench")
COLUMNS: tuple[tuple[str, pa.DataType], ...] = (
    ("schema", pa.int32()), ("op", pa.string()), ("impl", pa.string()), ("case", pa.string()),
    ("case_id", pa.string()), ("device", pa.string()), ("torch", pa.string()), ("backend_version", pa.string()),
    ("ts", pa.string()), ("ref_hash", pa.string()), ("impl_hash", pa.string()), ("status", pa.string()),
    ("reason", pa.string()), ("grad", pa.bool_()), ("benchmarked", pa.bool_()), ("bench_error", pa.string()),
    ("reps", pa.int32()),
) + tuple((name, pa.string()) for name in NESTED)
_ARROW_SCHEMA = pa.schema(list(COLUMNS))

_CONCLUSIVE = frozenset({"pass", "fail", "crash", "oom"})
_PROCESS_LOCK = threading.Lock()


def user_reports() -> Path:
    """The per-user report cache; the `v<schema>` segment keeps rows of other schemas apart."""
    root = os.getenv("POPCORN_CACHE_DIR")
    base = Path(root) if root is not None else Path(os.getenv("XDG_CACHE_HOME", Path.home() / ".cache")) / "popcorn"
    return base.expanduser() / f"v{SCHEMA}" / "reports"


def conclusive(record: Record) -> bool:
    """Does the row settle correctness for its case (pass, fail, crash or oom)?"""
    return record.result.status in _CONCLUSIVE


def unmeasured(record: Record | None, benchmark: bool = True) -> bool:
    """Should a run still produce this row? Absent, inconclusive (incl. oom), or, for timing, an untimed pass."""
    if record is None:
        return True
    status = record.result.status
    if status == "pass":
        return benchmark and not record.result.benchmarked
    return status not in ("fail", "crash")


def matching(expected: str | None, recorded: str | None) -> bool:
    """Fingerprints agree; code that cannot be hashed now (expected None) accepts any row."""
    return expected is None or expected == recorded


def _standing(record: Record, priority: int = 0) -> tuple[bool, str, int]:
    return conclusive(record), record.environment.ts, priority


def _row_order(key: tuple[Any, ...]) -> tuple[str, ...]:
    return tuple("" if part is None else str(part) for part in key)


class ReportFile:
    """One op's rows in one file; the suffix picks the format."""

    def __init__(self, path: Path | str) -> None:
        self.path = Path(path)

    @property
    def parquet(self) -> bool:
        return self.path.suffix == PUBLISHED

    def load(self) -> list[Record]:
        """Every row of the file; a file that is absent (or replaced mid-read) has none."""
        try:
            if self.parquet:
                rows = pq.read_table(self.path).to_pylist()
                for row in rows:
                    for name in NESTED:
                        row[name] = json.loads(row[name]) if row[name] is not None else {}
            else:
                rows = [json.loads(line) for line in self.path.read_text().splitlines() if line.strip()]
        except FileNotFoundError:
            return []
        return [Record.from_dict(row) for row in rows]

    def _encode(self, records: list[Record], target: Path) -> None:
        if self.parquet:
            rows = []
            for record in records:
                row = record.to_dict()
                rows.append({**row, **{name: json.dumps(row.get(name) or {}, sort_keys=True) for name in NESTED}})
            pq.write_table(pa.Table.from_pylist(rows, schema=_ARROW_SCHEMA), target, compression="zstd")
        else:
            target.write_text("".join(json.dumps(r.to_dict(), sort_keys=True) + "\n" for r in records))

    def save(self, records: list[Record]) -> None:
        """Replace the file's rows atomically (a temporary file, then a rename)."""
        temporary = self.path.with_name(f".{self.path.name}.{os.getpid()}.{threading.get_ident()}.tmp")
        try:
            self._encode(records, temporary)
            os.replace(temporary, self.path)
        finally:
            temporary.unlink(missing_ok=True)

    @contextmanager
    def locked(self) -> Iterator[None]:
        """Exclusive access across threads (a process lock) and processes (flock on a side file)."""
        with _PROCESS_LOCK, open(self.path.with_name(self.path.name + ".lock"), "a") as handle:
            if fcntl is not None:
                fcntl.flock(handle, fcntl.LOCK_EX)
            try:
                yield
            finally:
                if fcntl is not None:
                    fcntl.flock(handle, fcntl.LOCK_UN)


def read_file(path: Path | str) -> list[Record]:
    return ReportFile(path).load()


def read(directory: Path | str) -> list[Record]:
    """Every row of a reports directory: the Parquet files first, then the JSONL ones, each sorted by name."""
    directory = Path(directory)
    files = sorted(directory.glob(f"*{PUBLISHED}")) + sorted(directory.glob(f"*{SCRATCH}"))
    return [record for path in files for record in read_file(path)]


def bundled_path(directory: Path | str, op: str) -> Path:
    """Where an op's published rows are: its Parquet file when there is one, else its JSONL file."""
    parquet = Path(directory) / f"{op}{PUBLISHED}"
    return parquet if parquet.exists() else parquet.with_suffix(SCRATCH)


def _upsert(kept: dict[tuple[Any, ...], Record], record: Record) -> None:
    held = kept.get(record.key)
    if held is None or _standing(record) >= _standing(held):
        kept[record.key] = record


def write(records: Iterable[Record], directory: Path | str, suffix: str = SCRATCH) -> None:
    """Merge rows into `<op><suffix>` files by key (see the module docstring for which row stays)."""
    directory = Path(directory)
    directory.mkdir(parents=True, exist_ok=True)
    by_op: dict[str, list[Record]] = defaultdict(list)
    for record in records:
        by_op[record.op].append(record)
    for op in sorted(by_op):
        target = ReportFile(directory / f"{op}{suffix}")
        with target.locked():
            kept: dict[tuple[Any, ...], Record] = {}
            for record in target.load() + by_op[op]:
                _upsert(kept, record)
            target.save([kept[key] for key in sorted(kept, key=_row_order)])


def scrub(directory: Path | str, drop: Callable[[Record], bool]) -> int:
    """Remove the rows `drop` selects from every report file of a directory; returns how many went.

    A file left without rows is deleted. (Popcorn uses this for bookkeeping rows
    that never became measurements, bench/store.py:382-409.)
    """
    removed = 0
    directory = Path(directory)
    for path in sorted(directory.glob(f"*{PUBLISHED}")) + sorted(directory.glob(f"*{SCRATCH}")):
        target = ReportFile(path)
        with target.locked():
            rows = target.load()
            kept = [row for row in rows if not drop(row)]
            if len(kept) == len(rows):
                continue
            removed += len(rows) - len(kept)
            if kept:
                target.save(kept)
            else:
                path.unlink()
    return removed


def publish(directory: Path | str, ops: Iterable[str] | None = None, user: Path | str | None = None) -> int:
    """Merge the user cache's rows (all ops, or `ops`) into `<op>.parquet` files in `directory`.

    This is how rows measured on an MI355X become a reports directory that
    Popcorn can read. Returns the number of rows offered.
    """
    source = Path(user) if user is not None else user_reports()
    wanted = None if ops is None else set(ops)
    rows = [r for path in sorted(source.glob(f"*{SCRATCH}")) for r in read_file(path)
            if wanted is None or r.op in wanted]
    write(rows, directory, PUBLISHED)
    return len(rows)


class Reports:
    """The rows dispatch reads for an op: published rows merged with the user cache.

    Directories left as None are looked up on every read (`BUNDLED_REPORTS`,
    `user_reports()`), so pointing the cache elsewhere takes effect at once.
    """

    def __init__(self, bundled: Path | str | None = None, user: Path | str | None = None) -> None:
        self._bundled = None if bundled is None else Path(bundled)
        self._user = None if user is None else Path(user)

    @property
    def bundled(self) -> Path:
        return self._bundled if self._bundled is not None else BUNDLED_REPORTS

    @property
    def user(self) -> Path:
        return self._user if self._user is not None else user_reports()

    def rows(self, op: str) -> tuple[Record, ...]:
        """One row per key across the published file and the user cache; on a tie the user cache wins."""
        sources = [bundled_path(self.bundled, op), self.user / f"{op}{SCRATCH}"]
        best: dict[tuple[Any, ...], tuple[tuple[bool, str, int], Record]] = {}
        for priority, path in enumerate(dict.fromkeys(sources)):
            for record in read_file(path):
                key = record.key[1:]
                standing = _standing(record, priority)
                if key not in best or standing >= best[key][0]:
                    best[key] = (standing, record)
        return tuple(record for _, record in best.values())

    def write_user(self, records: Iterable[Record]) -> None:
        write(records, self.user)
