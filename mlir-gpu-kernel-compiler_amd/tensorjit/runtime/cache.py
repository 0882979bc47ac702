"""On-disk caches of the hip backend: compiled code objects and GEMM tile choices.

Both live under ``$TENSORJIT_CACHE_DIR``, else ``~/.cache/tensorjit`` -- the
reference's cache root (``tensorjit/runtime/cache.py:14-18``).

* ``CodeObjectCache``: one file per hipRTC build.  The file name is a digest of
  everything that decides the machine code: the source, the compile options,
  the device's full ``gcnArchName`` (feature flags included) and the toolchain
  (hipRTC and HIP runtime versions).  Upgrading ROCm or moving the cache to a
  different part therefore misses instead of loading stale code.
* ``AutotuneStore``: the reference's ``autotune.json`` format
  (``tensorjit/runtime/cache.py:28-61``): ``{key: {"config": {...}, "ms": t}}``.
  A write merges the new entry into what is on disk under an exclusive file
  lock, so processes tuning different shapes at the same time keep each
  other's results; a read picks up entries other processes wrote since.
  Keys name their gfx target (``hip|gfx950|matmul|...``), and a key missing from
  the user's file is looked up in the package's measured table for that
  target (``tensorjit/tuned/<target>.json``) unless ``TENSORJIT_RETUNE=1``.
"""
from __future__ import annotations

import fcntl
import hashlib
import json
import os
import tempfile
import threading
from contextlib import contextmanager
from pathlib import Path

TUNED_DIR = Path(__file__).resolve().parents[1] / "tuned"


def cache_dir() -> Path:
    root = os.environ.get("TENSORJIT_CACHE_DIR") or str(Path.home() / ".cache" / "tensorjit")
    path = Path(root)
    path.mkdir(parents=True, exist_ok=True)
    return path


def content_hash(*parts: str) -> str:
    """Hex digest naming a tuple of strings (each part length-prefixed, so ("ab", "c")
    and ("a", "bc") differ)."""
    h = hashlib.blake2b(digest_size=16)
    for part in parts:
        data = part.encode()
        h.update(len(data).to_bytes(8, "little"))
        h.update(data)
    return h.hexdigest()


def _replace_file(path: Path, data: bytes) -> None:
    """Write ``data`` to a temporary file beside ``path`` and rename it into place, so a
    reader sees either the old or the new file, never a partial one."""
    fd, tmp = tempfile.mkstemp(prefix=f".{path.name}.", dir=path.parent)
    try:
        with os.fdopen(fd, "wb") as f:
            f.write(data)
        os.replace(tmp, path)
    except BaseException:
        try:
            os.unlink(tmp)
        except OSError:
            pass
        raise


def packaged_entry(key: str) -> dict | None:
    """Entry for ``key`` in the package's measured table of the key's gfx target."""
    fields = key.split("|")
    if len(fields) < 2 or not fields[1]:
        return None
    table = TUNED_DIR / f"{fields[1]}.json"
    try:
        return json.loads(table.read_text()).get(key)
    except (OSError, ValueError):
        return None


class AutotuneStore:
    """Persisted GEMM tile choices: ``get(key)``, ``put(key, config, ms)``, ``clear()``."""

    _thread_lock = threading.Lock()

    def __init__(self, path: str | Path | None = None):
        p = Path(path) if path is not None else Path("autotune.json")
        self.path = p if p.is_absolute() else cache_dir() / p
        self._entries: dict[str, dict] = {}
        self._stamp: tuple[int, int] | None = None

    def _file_stamp(self) -> tuple[int, int] | None:
        try:
            st = self.path.stat()
        except OSError:
            return None
        return st.st_mtime_ns, st.st_size

    def _read_disk(self) -> dict[str, dict]:
        try:
            data = json.loads(self.path.read_text())
        except (OSError, ValueError):
            return {}
        return data if isinstance(data, dict) else {}

    def _refresh(self) -> None:
        stamp = self._file_stamp()
        if stamp != self._stamp:
            self._entries = self._read_disk()
            self._stamp = stamp

    @contextmanager
    def _exclusive(self):
        """This process's threads and other processes, one writer at a time."""
        self.path.parent.mkdir(parents=True, exist_ok=True)
        with self._thread_lock, open(self.path.with_name(self.path.name + ".lock"), "a+") as lk:
            fcntl.flock(lk, fcntl.LOCK_EX)
            try:
                yield
            finally:
                fcntl.flock(lk, fcntl.LOCK_UN)

    def get(self, key: str) -> dict | None:
        with self._thread_lock:
            self._refresh()
            hit = self._entries.get(key)
        if hit is None and os.environ.get("TENSORJIT_RETUNE") != "1":
            hit = packaged_entry(key)
        return hit

    def put(self, key: str, cfg: dict, ms: float) -> None:
        with self._exclusive():
            merged = self._read_disk()
            merged[key] = {"config": dict(cfg), "ms": float(ms)}
            _replace_file(self.path, json.dumps(merged, indent=1, sort_keys=True).encode())
            self._entries, self._stamp = merged, self._file_stamp()

    def clear(self) -> None:
        with self._exclusive():
            try:
                self.path.unlink()
            except FileNotFoundError:
                pass
            self._entries, self._stamp = {}, None


class CodeObjectCache:
    """hipRTC code objects on disk, keyed by source, options, target and toolchain."""

    def __init__(self, target: str, toolchain: str):
        self.target = target
        self.toolchain = toolchain

    def path(self, source: str, opts: tuple[str, ...]) -> Path:
        digest = content_hash(source, "\n".join(opts), self.target, self.toolchain)
        gfx = self.target.split(":")[0]
        return cache_dir() / f"tj_hip_{gfx}_{digest}.co"

    def get(self, source: str, opts: tuple[str, ...]) -> bytes | None:
        try:
            return self.path(source, opts).read_bytes()
        except OSError:
            return None

    def put(self, source: str, opts: tuple[str, ...], code: bytes) -> None:
        _replace_file(self.path(source, opts), code)
