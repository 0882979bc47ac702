"""On-disk caches: HIP code objects and persisted GEMM autotune choices.

Root: ``$TENSORJIT_CACHE_DIR`` or ``~/.cache/tensorjit`` (ref
``tensorjit/runtime/cache.py:14-61``).  Code objects are keyed by the source
hash, the gfx target and the hipRTC version; autotune entries carry the
target in their key, so a cache directory can be shared between machines of
different architectures.
"""
from __future__ import annotations

import hashlib
import json
import os
import threading
from pathlib import Path


def cache_dir() -> Path:
    d = Path(os.environ.get("TENSORJIT_CACHE_DIR", Path.home() / ".cache" / "tensorjit"))
    d.mkdir(parents=True, exist_ok=True)
    return d


def content_hash(*parts: str) -> str:
    h = hashlib.sha256()
    for p in parts:
        h.update(p.encode())
        h.update(b"\0")
    return h.hexdigest()[:20]


def _atomic_write(path: Path, data: bytes) -> None:
    tmp = path.with_name(f"{path.name}.{os.getpid()}.{threading.get_ident()}.tmp")
    tmp.write_bytes(data)
    os.replace(tmp, path)


TUNED_DIR = Path(__file__).resolve().parents[1] / "tuned"


def _packaged(key: str) -> dict | None:
    """Read-only warm-start table shipped with the package (``tuned/<target>.json``),
    keyed like the user store; consulted when the user store has no entry."""
    parts = key.split("|")
    if len(parts) < 2:
        return None
    try:
        table = json.loads((TUNED_DIR / f"{parts[1]}.json").read_text())
    except (OSError, ValueError):
        return None
    return table.get(key)


class AutotuneStore:
    """JSON file of ``key -> {"config": ..., "ms": ...}``; writes are atomic renames.

    Lookups fall back to the package's warm-start table for the key's gfx target,
    so a fresh machine starts with measured tile choices instead of re-tuning;
    set ``TENSORJIT_RETUNE=1`` to ignore that table."""

    _lock = threading.Lock()

    def __init__(self, name: str = "autotune.json"):
        self.path = cache_dir() / name
        self._data: dict[str, dict] | None = None

    def _load(self) -> dict:
        if self._data is None:
            try:
                self._data = json.loads(self.path.read_text())
            except (OSError, ValueError):
                self._data = {}
        return self._data

    def get(self, key: str) -> dict | None:
        with self._lock:
            hit = self._load().get(key)
        if hit is None and os.environ.get("TENSORJIT_RETUNE") != "1":
            hit = _packaged(key)
        return hit

    def put(self, key: str, cfg: dict, ms: float) -> None:
        with self._lock:
            d = self._load()
            d[key] = {"config": cfg, "ms": ms}
            _atomic_write(self.path, json.dumps(d, indent=1, sort_keys=True).encode())

    def clear(self) -> None:
        with self._lock:
            self._data = {}
            if self.path.exists():
                self.path.unlink()


class CodeObjectCache:
    """Compiled gfx code objects, one file per (source, target, compiler) triple."""

    def __init__(self, target: str, compiler_tag: str):
        self.target = target
        self.compiler_tag = compiler_tag

    def path(self, source: str, opts: tuple[str, ...]) -> Path:
        key = content_hash(source, self.target, self.compiler_tag, " ".join(opts))
        return cache_dir() / f"tj_hip_{key}_{self.target}.co"

    def get(self, source: str, opts: tuple[str, ...]) -> bytes | None:
        p = self.path(source, opts)
        try:
            return p.read_bytes()
        except OSError:
            return None

    def put(self, source: str, opts: tuple[str, ...], code: bytes) -> None:
        _atomic_write(self.path(source, opts), code)
