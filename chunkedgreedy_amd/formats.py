"""Harness formats, so that permutations produced on the GPU flow into the
reference's tooling unchanged.

* Reorder hash: SHA-256 of the canonical JSON of (method, params[, env]),
  first 12 hex digits (reference spmatkit/spmatkit.py:267-307).  The paper's
  configurations hash to a609629886c6 (sporder-csg), eefae4eb9269 (sporder-cg)
  and 685c3b160263 (ORIGIN), as configs/paper.yaml:6-15 lists.
* ``.perm.npz``: ``<root>/<method>/<matrix>_<hash>.perm.npz`` holding
  ``row_perm`` (int64, new2old), ``matrix``, ``reorder_method``,
  ``params_json``, ``reorder_hash``, ``env_json``, ``created_at`` and
  optionally ``source`` (spmatkit.py:947-1100).  Every field is a plain numpy
  array (strings as unicode scalars), so ``numpy.load`` reads it without
  pickle.
* Reorder-bench CSV: the 22 columns of bench/reorder/reorder_bench/
  results.py:14-37, one row per (matrix, method, hash), with the structure
  metrics bandwidth / profile / tc_h / tc_w / tc_num / tc_fill_rate
  (spmatkit.py:1704-1717, 1974-1995, 2037-2060) computed on the GPU by
  ``quality.reorder_bench_metrics``.
"""

from __future__ import annotations

import csv
import hashlib
import json
import os
from datetime import datetime, timezone
from pathlib import Path
from typing import Any

import numpy as np

PERM_SUFFIX = ".perm.npz"
ORIGIN_METHOD = "ORIGIN"

RESULT_COLUMNS = [
    "matrix", "reorder_method", "params_json", "reorder_hash", "effective_params_json",
    "env_json", "success", "error", "load_matrix_ms", "prep_ms", "reorder_time_ms",
    "perm_trans_ms", "eval_time_ms", "timing_breakdown_json", "bandwidth", "profile", "tc_h",
    "tc_w", "tc_num", "tc_fill_rate", "source_commit", "timestamp",
]


def _normalize(value):
    # bool stays bool; integral numbers become int; other floats stay float.
    if isinstance(value, (bool, np.bool_)):
        return bool(value)
    if isinstance(value, (int, np.integer)):
        return int(value)
    if isinstance(value, (float, np.floating)):
        return int(value) if value == int(value) else float(value)
    if isinstance(value, str):
        return value
    raise TypeError(f"cannot hash a parameter of type {type(value).__name__}")


def canonicalize_params(params: dict) -> str:
    """Canonical JSON of a params dict: sorted keys, no spaces."""
    if not isinstance(params, dict):
        raise TypeError(f"reorder parameters: expected a dict, got {type(params).__name__}")
    return json.dumps({k: _normalize(params[k]) for k in sorted(params)}, sort_keys=True,
                      separators=(",", ":"))


def compute_reorder_hash(reorder_method: str, params: dict, env: dict | None = None) -> str:
    """12-hex-digit identity of a reorder configuration."""
    env = env or {}
    if not isinstance(env, dict):
        raise TypeError(f"reorder environment: expected a dict, got {type(env).__name__}")
    payload = {"method": reorder_method, "params": json.loads(canonicalize_params(params))}
    if env:
        payload["env"] = json.loads(canonicalize_params(env))
    text = json.dumps(payload, sort_keys=True, separators=(",", ":"))
    return hashlib.sha256(text.encode("utf-8")).hexdigest()[:12]


def get_perm_path(root, matrix: str, reorder_method: str, reorder_hash: str) -> Path:
    return Path(root) / reorder_method / f"{matrix}_{reorder_hash}{PERM_SUFFIX}"


def validate_row_perm(row_perm, nrows: int) -> np.ndarray:
    perm = np.asarray(row_perm, dtype=np.int64)
    if perm.ndim != 1:
        raise ValueError(f"row permutation has {perm.ndim} dimensions; one is required")
    if perm.shape[0] != nrows:
        raise ValueError(f"row permutation holds {perm.shape[0]} entries for a matrix of {nrows} rows")
    seen = np.zeros(nrows, dtype=bool)
    if perm.size and (perm.min() < 0 or perm.max() >= nrows):
        raise ValueError("row_perm must hold each row index 0..nrows-1 exactly once")
    seen[perm] = True
    if not seen.all():
        raise ValueError("row_perm must hold each row index 0..nrows-1 exactly once")
    return perm


def save_reorder_perm(root, matrix: str, reorder_method: str, params: dict, row_perm, *,
                      env: dict | None = None, source: str | None = None) -> Path:
    """Write <root>/<method>/<matrix>_<hash>.perm.npz atomically; returns the path."""
    if reorder_method == ORIGIN_METHOD:
        raise ValueError("ORIGIN has no permutation to store")
    perm = validate_row_perm(row_perm, int(np.asarray(row_perm).shape[0]))
    env = env or {}
    reorder_hash = compute_reorder_hash(reorder_method, params, env)
    path = get_perm_path(root, matrix, reorder_method, reorder_hash)
    path.parent.mkdir(parents=True, exist_ok=True)
    fields = {
        "row_perm": perm,
        "matrix": np.array(matrix),
        "reorder_method": np.array(reorder_method),
        "params_json": np.array(canonicalize_params(params)),
        "reorder_hash": np.array(reorder_hash),
        "env_json": np.array(canonicalize_params(env)),
        "created_at": np.array(datetime.now(timezone.utc).isoformat(timespec="seconds")),
    }
    if source is not None:
        fields["source"] = np.array(source)
    tmp = path.with_suffix(".perm.tmp.npz")
    try:
        np.savez(tmp, **fields)
        tmp.replace(path)
    finally:
        if tmp.exists():
            tmp.unlink()
    return path


def load_reorder_perm(path, nrows: int | None = None) -> np.ndarray:
    """row_perm (int64, new2old) of a .perm.npz; validated when nrows is given."""
    with np.load(path, allow_pickle=False) as archive:
        perm = np.asarray(archive["row_perm"], dtype=np.int64)
    if nrows is not None:
        validate_row_perm(perm, nrows)
    return perm


def reorder_result_row(matrix: str, reorder_method: str, params: dict, result, metrics: dict,
                       *, env: dict | None = None, load_matrix_ms: float = 0.0,
                       eval_ms: float = 0.0, source_commit: str = "") -> dict[str, Any]:
    """One reorder-bench CSV row from a ReorderResult (harness.ReorderResult) and the
    structure metrics (bench/reorder/reorder_bench/run_bench.py:250-305)."""
    env = env or {}
    row = {
        "timestamp": datetime.now(timezone.utc).isoformat(timespec="seconds"),
        "matrix": matrix,
        "reorder_method": reorder_method,
        "params_json": canonicalize_params(params),
        "reorder_hash": compute_reorder_hash(reorder_method, params, env),
        "effective_params_json": json.dumps(result.effective_params, sort_keys=True),
        "env_json": canonicalize_params(env),
        "success": "1",
        "error": "",
        "load_matrix_ms": f"{load_matrix_ms:.4f}",
        "prep_ms": f"{result.prep_time_ms:.4f}",
        "reorder_time_ms": f"{result.reorder_time_ms:.4f}",
        "perm_trans_ms": f"{result.perm_trans_ms:.4f}",
        "eval_time_ms": f"{eval_ms:.4f}",
        "timing_breakdown_json": json.dumps(result.timing_breakdown, sort_keys=True),
        "source_commit": source_commit,
    }
    for key in ("bandwidth", "profile", "tc_h", "tc_w", "tc_num", "tc_fill_rate"):
        if key in metrics:
            row[key] = metrics[key]
    return row


def write_result_row(path, row: dict[str, Any]) -> None:
    """Append a row to a reorder-bench CSV, writing the header for a new file and
    refusing a file whose header differs (results.py:88-97)."""
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    new = not path.exists() or path.stat().st_size == 0
    if not new:
        with path.open(newline="", encoding="utf-8") as fh:
            header = next(csv.reader(fh), None)
        if header != RESULT_COLUMNS:
            raise ValueError(f"{path} has an outdated CSV header; write to a new file")
    with path.open("a", newline="", encoding="utf-8") as fh:
        writer = csv.DictWriter(fh, fieldnames=RESULT_COLUMNS, extrasaction="ignore")
        if new:
            writer.writeheader()
        writer.writerow({c: row.get(c, "") for c in RESULT_COLUMNS})
        fh.flush()
        os.fsync(fh.fileno())
