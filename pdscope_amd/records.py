"""Run records in the reference's file layout, for side-by-side comparison.

A measured run writes, next to its ``result.json``:

* ``manifest.json`` -- how and where the run was made: command line and
  configuration, host, Python/package versions, git commit and worktree
  status, device and CPU descriptions, and an archive of the source files
  with their hashes (``source.zip``); written with status "running" when the
  run starts and completed (status, finish time, result hash) or marked failed
  when it ends (the manifest of benchmarks/harness.py:125-183 and the run
  wrapper of benchmarks/pdscope_compare.py:828-850);
* ``cases.json`` -- the case specifications;
* ``requests.jsonl`` -- one JSON line per finished request (case): timings,
  generated ids, ledger counters, memory figures and the hash of its trace
  (the request record of pdscope_compare.py:390-436);
* ``traces/<case_id>.json.gz`` -- the runtime's per-layer trace rows
  (expertbench/pdscope_runtime.py:492-512);
* ``result.json`` -- every request plus run-wide identity and environment
  (schema version 2, pdscope_compare.py:436-470);
* ``failure.txt`` -- the traceback when the run failed.

The key names are the reference's, so the same tooling can read both; where
a field names NVIDIA tooling the record carries the ROCm equivalent under its
own name (``rocm_smi``) and the reference's key holds None.
"""
from __future__ import annotations

import gzip
import hashlib
import json
import math
import os
import platform
import resource
import subprocess
import sys
import time
import traceback
import zipfile
from datetime import datetime, timezone
from pathlib import Path

REPO = Path(__file__).resolve().parent.parent
SOURCE_SUFFIXES = (".py", ".hip", ".h", ".c", ".cpp")
ENV_KEYS = ("OMP_NUM_THREADS", "MKL_NUM_THREADS", "HIP_VISIBLE_DEVICES", "ROCR_VISIBLE_DEVICES",
            "CUDA_VISIBLE_DEVICES", "LD_LIBRARY_PATH", "PYTHONPATH", "PYTHONHOME", "PYTORCH_CUDA_ALLOC_CONF",
            "PYTORCH_ALLOC_CONF", "PYTHONHASHSEED", "HSA_ENABLE_IPC_MODE_LEGACY")


def sha256_bytes(data):
    return hashlib.sha256(data).hexdigest()


def sha256_file(path):
    return sha256_bytes(Path(path).read_bytes())


def peak_rss_bytes():
    return resource.getrusage(resource.RUSAGE_SELF).ru_maxrss * 1024


def run_command(argv, timeout=30):
    """argv's exit status and output (the program may be absent)."""
    try:
        p = subprocess.run(argv, text=True, capture_output=True, timeout=timeout)
        return dict(argv=argv, returncode=p.returncode, stdout=p.stdout, stderr=p.stderr)
    except (OSError, subprocess.TimeoutExpired) as err:
        return dict(argv=argv, returncode=None, stdout="", stderr=f"{type(err).__name__}: {err}")


def phase_metrics(input_tokens, token_ready_seconds):
    """Request timing from the completion time of every generated token
    (seconds from the start of the request).  The first token closes the
    prefill; decode covers the forwards after it (the definitions of
    pdscope_compare.py:129-141)."""
    ready = list(token_ready_seconds)
    if type(input_tokens) is not int or input_tokens < 1 or len(ready) < 2:
        raise ValueError("metrics need a positive prompt length and at least two generated tokens")
    if any(not isinstance(t, (int, float)) or not math.isfinite(t) or t <= 0 for t in ready):
        raise ValueError("token completion times must be positive and finite")
    if any(b <= a for a, b in zip(ready, ready[1:])):
        raise ValueError("token completion times must increase")
    prefill = ready[0]
    decode = ready[-1] - prefill
    forwards = len(ready) - 1
    return dict(input_tokens=input_tokens, output_tokens=len(ready), decode_forwards=forwards,
                prefill_seconds=prefill, decode_seconds=decode, request_output_seconds=ready[-1],
                prefill_tokens_per_second=input_tokens / prefill, decode_tokens_per_second=forwards / decode,
                end_to_end_output_tokens_per_second=len(ready) / ready[-1], decode_tpot_seconds=decode / forwards,
                scope="first generated token belongs to prefill; decode counts actual subsequent forwards")


def _source_files(root):
    listed = run_command(["git", "-C", str(root), "ls-files", "-z"])
    names = [n for n in listed["stdout"].split("\0") if n] if listed["returncode"] == 0 else []
    if not names:  # not a git checkout: the package and oracle sources on disk
        names = [str(p.relative_to(root)) for d in ("pdscope_amd", "oracle", "include") for p in (root / d).rglob("*")
                 if p.is_file()]
    return sorted(n for n in set(names) if n.endswith(SOURCE_SUFFIXES) and (root / n).is_file()
                  and not n.startswith("_work/"))


def capture_manifest(output_dir, *, entry, argv, config, root=REPO):
    """The run's manifest, with the source archive written to output_dir/source.zip."""
    import importlib.metadata
    output_dir = Path(output_dir)
    versions = {}
    for name in ("torch", "transformers", "safetensors", "numpy"):
        try:
            versions[name] = importlib.metadata.version(name)
        except importlib.metadata.PackageNotFoundError:
            versions[name] = None
    members = {}
    archive = output_dir / "source.zip"
    with zipfile.ZipFile(archive, "x", compression=zipfile.ZIP_DEFLATED) as z:
        for name in _source_files(root):
            data = (root / name).read_bytes()
            z.writestr(name, data)
            members[name] = sha256_bytes(data)
    library = root / "pdscope_amd" / "libpdscope_moe.so"
    native = dict(source_hashes={n: h for n, h in members.items() if n.startswith(("pdscope_amd/csrc/", "include/"))},
                  artifacts=[dict(path=str(library), role="gfx950 kernel library (C-ABI)", sha256=sha256_file(library),
                                  bytes=library.stat().st_size)] if library.is_file() else [])
    try:
        cmdline = Path("/proc/self/cmdline").read_bytes().decode().split("\0")[:-1]
    except OSError:
        cmdline = list(sys.argv)
    return dict(schema_version=1, entry=entry, argv=list(argv),
                config={k: str(v) if isinstance(v, Path) else v for k, v in dict(config).items()},
                started_at=datetime.now(timezone.utc).isoformat(), pid=os.getpid(), cwd=os.getcwd(),
                python=sys.version, executable=sys.executable, host=platform.node(), platform=platform.platform(),
                package_versions=versions, process_argv=cmdline, affinity=sorted(os.sched_getaffinity(0)),
                env={k: os.environ.get(k) for k in ENV_KEYS},
                git_commit=run_command(["git", "-C", str(root), "rev-parse", "HEAD"]),
                git_status=run_command(["git", "-C", str(root), "status", "--short", "--", "."]),
                nvidia_smi=None, rocm_smi=run_command(["rocm-smi", "--showproductname", "--showmeminfo", "vram"]),
                lscpu=run_command(["lscpu", "-J"]),
                source_archive=dict(path=archive.name, sha256=sha256_file(archive), members=members,
                                    includes_dirty_worktree_bytes=True),
                native_prefetch_build=native, status="running")


class RunRecorder:
    """Writes one run's files (see the module docstring) under the directory of
    `result_path`, which must not exist yet."""

    def __init__(self, result_path, *, entry, argv, config, root=REPO):
        self.result_path = Path(result_path).resolve()
        if self.result_path.exists():
            raise FileExistsError(f"refusing to overwrite an existing result: {self.result_path}")
        self.dir = self.result_path.parent
        self.dir.mkdir(parents=True, exist_ok=True)
        self.started = time.monotonic()
        self.manifest = capture_manifest(self.dir, entry=entry, argv=argv, config=config, root=root)
        self._write_manifest()
        self.requests = []

    def _write_manifest(self):
        (self.dir / "manifest.json").write_text(json.dumps(self.manifest, indent=2) + "\n")

    def cases(self, specs):
        (self.dir / "cases.json").write_text(json.dumps(dict(schema_version=1, cases=list(specs)), indent=2) + "\n")

    def trace(self, case_id, rows):
        """Store a request's per-layer trace rows; returns the trace record."""
        path = self.dir / "traces" / f"{case_id}.json.gz"
        path.parent.mkdir(exist_ok=True)
        with gzip.open(path, "wt") as f:
            json.dump(rows, f, separators=(",", ":"), default=_jsonable)
        return dict(path=str(path.relative_to(self.dir)), sha256=sha256_file(path))

    def request(self, record):
        """Append one finished request to requests.jsonl."""
        with (self.dir / "requests.jsonl").open("a") as f:
            f.write(json.dumps(record, separators=(",", ":"), default=_jsonable) + "\n")
        self.requests.append(record)

    def finish(self, result):
        self.result_path.write_text(json.dumps(result, indent=2, default=_jsonable) + "\n")
        self.manifest.update(status="completed", result_sha256=sha256_file(self.result_path))
        self._close()

    def fail(self, exc):
        self.manifest.update(status="failed", error_type=type(exc).__name__, error=str(exc))
        (self.dir / "failure.txt").write_text("".join(traceback.format_exception(type(exc), exc, exc.__traceback__)))
        self._close()

    def _close(self):
        self.manifest.update(finished_at=datetime.now(timezone.utc).isoformat(),
                             runner_seconds=time.monotonic() - self.started, host_peak_rss_bytes=peak_rss_bytes())
        self._write_manifest()


def _jsonable(value):
    """JSON form of the non-JSON values trace rows hold (ExpertKey, tuples as keys are pre-converted)."""
    if hasattr(value, "__dataclass_fields__"):
        return {k: getattr(value, k) for k in value.__dataclass_fields__}
    if isinstance(value, (set, frozenset)):
        return sorted(value)
    return str(value)


def trace_row_json(row):
    """A trace row with its integer-keyed dicts made JSON-stable (str keys)."""
    def fix(v):
        if isinstance(v, dict):
            return {str(k): fix(x) for k, x in v.items()}
        if isinstance(v, (list, tuple)):
            return [fix(x) for x in v]
        return v
    return fix(row)
