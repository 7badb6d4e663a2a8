"""The training-curve artefact in the reference's ``.riglog`` container.

Layout (``docs/RIGLOG_FORMAT.md:31-63``; writer ``rig/logpack.py``), all
little-endian:

    offset 0       8 bytes   magic  b"RIGLOG\\x00\\x01"
    offset 8       int32     column_count         (4 bytes padding after it)
    offset 16      int64     tokens_per_step
    offset 24      float64   flops_per_token
    offset 32      n x 24    column table: int32 metric_id, int32 scope_id,
                             int32 layer (-1: not layered), int32 index
                             (-1: unused), int64 element_count
    offset 32+24n  m x (4+4n) records: int32 step, n x float32 values

Column ids are the reference registry's permanent ids (``rig/metrics.py:80-86``
for the run-level scalars, ``:136-140`` for the scopes; snapshot
``rig/registry.txt``).  The training curve is three ``overall`` columns --
``train_loss``, ``learning_rate``, ``grad_norm`` -- one record per optimizer
step (``rig/runlog.py:133-175``, ``:257-302``), which is exactly the row layout
of ``GPTTrainer.history``.  ``tokens_processed`` and ``cumulative_flops`` are
not stored; a reader derives them from the step in int64 / float64.
"""

from __future__ import annotations

import csv
import json
import math
import os
import struct
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Iterable, Mapping, Sequence

import numpy as np

MAGIC = b"RIGLOG\x00\x01"
SUFFIX = ".riglog"
TRAINING_LOG_NAME = "training" + SUFFIX
# Run-directory names and the result event (rig/runlog.py:36-39, :118-126; rig/harness/validation.py:17-18).
CHECKPOINT_NAME = "checkpoint.npz"
VALIDATION_CSV_NAME = "validation.csv"
RESULT_NAME = "metrics.json"
RESULT_PREFIX = "RIG_RESULT="
SCHEMA_VERSION = 1

# Registry ids (permanent in the reference; only the ones this build writes or derives).
METRIC_IDS = {"step": 1, "tokens_processed": 2, "cumulative_flops": 3, "train_loss": 4, "learning_rate": 5,
              "grad_norm": 6}
SCOPE_IDS = {"overall": 1, "embeddings": 2, "unembedding": 3, "block": 4, "final_norm": 5}
TRAINING_COLUMNS = ("train_loss", "learning_rate", "grad_norm")

_HEADER = struct.Struct("<i4xqd")   # column_count, pad, tokens_per_step, flops_per_token
_COLUMN = struct.Struct("<iiiiq")   # metric_id, scope_id, layer, index, element_count
_COLUMN_DTYPE = np.dtype([("metric_id", "<i4"), ("scope_id", "<i4"), ("layer", "<i4"), ("index", "<i4"),
                          ("element_count", "<i8")])


class LogError(ValueError):
    """A file that is not, or is no longer, a readable ``.riglog``."""


@dataclass(frozen=True)
class Column:
    metric_id: int
    scope_id: int = SCOPE_IDS["overall"]
    layer: int = -1
    index: int = -1
    element_count: int = 0


def training_columns() -> tuple[Column, ...]:
    return tuple(Column(METRIC_IDS[name]) for name in TRAINING_COLUMNS)


def header_size(columns: int) -> int:
    return len(MAGIC) + _HEADER.size + columns * _COLUMN.size


def record_size(columns: int) -> int:
    return 4 + 4 * columns


class LogWriter:
    """Writes the header on open and one fixed-width record per ``append``,
    flushed each time, so the file is a valid log after every append."""

    def __init__(self, path, columns: Sequence[Column], *, tokens_per_step: int, flops_per_token: float = 1.0):
        columns = tuple(columns)
        if not columns:
            raise ValueError("a log needs at least one column")
        if int(tokens_per_step) <= 0:
            raise ValueError(f"tokens_per_step must be positive, got {tokens_per_step}")
        if not float(flops_per_token) > 0.0:
            raise ValueError(f"flops_per_token must be positive, got {flops_per_token}")
        self.columns = columns
        self._last_step = None
        self._handle = open(path, "wb")
        self._handle.write(MAGIC)
        self._handle.write(_HEADER.pack(len(columns), int(tokens_per_step), float(flops_per_token)))
        for c in columns:
            self._handle.write(_COLUMN.pack(c.metric_id, c.scope_id, c.layer, c.index, c.element_count))
        self._handle.flush()

    def append(self, step: int, values: Iterable[float]) -> None:
        row = np.asarray(list(values), dtype="<f4")
        if row.shape != (len(self.columns),):
            raise ValueError(f"expected {len(self.columns)} values, got {row.shape}")
        step = int(step)
        if self._last_step is not None and step <= self._last_step:
            raise ValueError(f"steps must increase: {step} after {self._last_step}")
        self._last_step = step
        self._handle.write(struct.pack("<i", step) + row.tobytes())
        self._handle.flush()

    def close(self) -> None:
        self._handle.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


@dataclass
class Log:
    columns: tuple[Column, ...]
    steps: np.ndarray
    values: np.ndarray
    tokens_per_step: int
    flops_per_token: float

    def axis(self, name: str) -> np.ndarray:
        """``step``, ``tokens_processed`` (int64) or ``cumulative_flops`` (float64), derived from the step."""

        if name == "step":
            return self.steps
        if name == "tokens_processed":
            return self.steps.astype(np.int64) * np.int64(self.tokens_per_step)
        if name == "cumulative_flops":
            return (self.steps.astype(np.int64) * np.int64(self.tokens_per_step)).astype(np.float64) \
                * self.flops_per_token
        raise KeyError(f"{name!r} is not a derived axis")

    def series(self, metric: str, scope: str = "overall", layer: int = -1) -> np.ndarray | None:
        want = (METRIC_IDS[metric], SCOPE_IDS[scope], layer)
        for i, c in enumerate(self.columns):
            if (c.metric_id, c.scope_id, c.layer) == want:
                return self.values[:, i]
        return None


def read_log(path) -> Log:
    """Whole-file read; a partial trailing record (an interrupted writer) is dropped."""

    raw = Path(path).read_bytes()
    if not raw.startswith(MAGIC):
        raise LogError(f"{path} is not a .riglog (bad magic)")
    if len(raw) < len(MAGIC) + _HEADER.size:
        raise LogError(f"{path} is truncated inside its header")
    n, tokens_per_step, flops_per_token = _HEADER.unpack_from(raw, len(MAGIC))
    if n <= 0:
        raise LogError(f"{path} declares {n} columns")
    start = header_size(n)
    if len(raw) < start:
        raise LogError(f"{path} is truncated inside its column table")
    table = np.frombuffer(raw, dtype=_COLUMN_DTYPE, count=n, offset=len(MAGIC) + _HEADER.size)
    columns = tuple(Column(int(r["metric_id"]), int(r["scope_id"]), int(r["layer"]), int(r["index"]),
                           int(r["element_count"])) for r in table)
    stride = record_size(n)
    count = (len(raw) - start) // stride
    body = np.frombuffer(raw, dtype=np.uint8, count=count * stride, offset=start).reshape(count, stride)
    steps = np.ascontiguousarray(body[:, :4]).view("<i4").reshape(count)
    values = np.ascontiguousarray(body[:, 4:]).view("<f4").reshape(count, n)
    return Log(columns, steps, values, int(tokens_per_step), float(flops_per_token))


def write_training_log(output_dir, history: np.ndarray, *, tokens_per_step: int, final_step: int,
                       flops_per_token: float | None = None, columns: Sequence[Column] | None = None) -> Path:
    """Write ``training.riglog`` with one record per optimizer step 1..final_step
    (``rig/runlog.py:257-302``).

    ``history`` is the ``[horizon, len(columns)]`` step buffer; rows past
    ``final_step`` (an early stop leaves them zero) are dropped.  Without a FLOP
    count the header carries 1.0 and the FLOP axis is not meaningful.  The file
    goes through a temporary name and ``os.replace``, so the destination is the
    previous file or the complete new one, never a mix."""

    history = np.asarray(history, dtype=np.float32)
    resolved = training_columns() if columns is None else tuple(columns)
    if history.ndim == 2 and history.shape[0] > final_step:
        history = history[:final_step]
    if history.shape != (final_step, len(resolved)):
        raise ValueError(f"training history has shape {history.shape}; expected {(final_step, len(resolved))}")
    if flops_per_token is not None and not flops_per_token > 0:
        raise ValueError("flops_per_token must be positive when provided")
    out = Path(output_dir)
    out.mkdir(parents=True, exist_ok=True)
    destination = out / TRAINING_LOG_NAME
    temporary = out / f".{TRAINING_LOG_NAME}.tmp"
    with LogWriter(temporary, resolved, tokens_per_step=tokens_per_step,
                   flops_per_token=float(flops_per_token or 1.0)) as writer:
        for i, row in enumerate(history, 1):
            writer.append(i, row)
    os.replace(temporary, destination)
    return destination


# --- the rest of a run directory ---------------------------------------------------------------

def finite_metric(name: str, value: float, *, positive: bool = False) -> float:
    """A result metric as a float, refused if NaN/inf, negative, or (``positive``) zero (``rig/mesh.py:214-223``)."""

    value = float(value)
    if not math.isfinite(value) or value < 0.0 or (positive and value == 0.0):
        raise FloatingPointError(f"{name} must be finite and {'positive' if positive else 'nonnegative'}, "
                                 f"got {value!r}")
    return value


def _replace_atomically(destination: Path, write) -> Path:
    temporary = destination.parent / f".{destination.name}.tmp"
    with temporary.open("wb") as handle:
        write(handle)
        handle.flush()
        os.fsync(handle.fileno())
    os.replace(temporary, destination)
    return destination


def write_result(output_dir, result: Mapping[str, Any]) -> Path:
    """``metrics.json``: indented, sorted keys, no NaN, trailing newline, atomic (``rig/runlog.py:118-126``)."""

    text = json.dumps(result, indent=2, sort_keys=True, allow_nan=False) + "\n"
    out = Path(output_dir)
    out.mkdir(parents=True, exist_ok=True)
    return _replace_atomically(out / RESULT_NAME, lambda h: h.write(text.encode("utf-8")))


def result_line(result: Mapping[str, Any]) -> str:
    """The final stdout line a harness parses: ``RIG_RESULT=`` + compact sorted JSON
    (``recipes/reference/train.py:2411-2415``; ``rig/harness/validation.py:28-47``)."""

    return RESULT_PREFIX + json.dumps(result, sort_keys=True, separators=(",", ":"), allow_nan=False)


@dataclass(frozen=True)
class ValidationRow:
    """One validation score (``rig/runlog.py:43-53``)."""

    step: int
    tokens_processed: int
    kind: str
    domain: str
    validation_tokens: int
    validation_loss: float
    perplexity: float
    validation_seconds: float
    canonical: bool


VALIDATION_CSV_HEADER = ("step", "tokens_processed", "kind", "domain", "validation_tokens", "validation_loss",
                         "perplexity", "validation_seconds", "canonical")


def write_validation_csv(output_dir, rows: Sequence[ValidationRow]) -> Path:
    """``validation.csv`` with exactly one canonical ``fineweb`` row (``rig/runlog.py:355-413``)."""

    canonical = [r for r in rows if r.canonical]
    if len(canonical) != 1 or canonical[0].kind != "fineweb":
        raise ValueError("validation history must contain one canonical in-distribution row")
    lines = []

    class _Sink:
        def write(self, text):
            lines.append(text)

    writer = csv.writer(_Sink(), lineterminator="\n")
    writer.writerow(VALIDATION_CSV_HEADER)
    for r in rows:
        writer.writerow((int(r.step), int(r.tokens_processed), r.kind, r.domain, int(r.validation_tokens),
                         float(r.validation_loss), float(r.perplexity), float(r.validation_seconds),
                         "true" if r.canonical else "false"))
    out = Path(output_dir)
    out.mkdir(parents=True, exist_ok=True)
    return _replace_atomically(out / VALIDATION_CSV_NAME, lambda h: h.write("".join(lines).encode("utf-8")))


def save_checkpoint(output_dir, params: Mapping[str, np.ndarray], metadata: Mapping[str, Any]) -> Path:
    """``checkpoint.npz``: every parameter under ``params/<path>`` plus the
    sorted-key JSON ``metadata`` as a uint8 array named ``metadata.json``
    (``rig/runlog.py:96-115``, key paths as ``rig/nn.py:63-77`` flattens them)."""

    arrays = {f"params/{path}": np.asarray(value) for path, value in sorted(params.items())}
    arrays["metadata.json"] = np.frombuffer(json.dumps(metadata, sort_keys=True).encode("utf-8"), dtype=np.uint8)
    out = Path(output_dir)
    out.mkdir(parents=True, exist_ok=True)
    return _replace_atomically(out / CHECKPOINT_NAME, lambda h: np.savez(h, **arrays))
