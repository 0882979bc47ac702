"""Autotune store and the packaged warm-start tile table (CPU only)."""
import json

import pytest

from tensorjit.backends import hip_gemm
from tensorjit.ir import DType
from tensorjit.runtime import cache
from tensorjit.runtime.autotune import MatmulConfig


def test_store_round_trip_and_atomic_file(tmp_path):
    store = cache.AutotuneStore(tmp_path / "autotune.json")
    key = "hip|gfx950|matmul|1x3x5x7|f32|tb0|epi0"
    assert store.get(key) is None
    cfg = MatmulConfig(64, 64, 16, 4, 2, 2, 32, 1).as_dict()
    store.put(key, cfg, 0.5)
    again = cache.AutotuneStore(tmp_path / "autotune.json")
    assert again.get(key) == {"config": cfg, "ms": 0.5}
    assert json.loads((tmp_path / "autotune.json").read_text())[key]["ms"] == 0.5


def test_packaged_table_is_a_fallback_only(tmp_path, monkeypatch):
    table = json.loads((cache.TUNED_DIR / "gfx950.json").read_text())
    key = next(iter(table))
    store = cache.AutotuneStore(tmp_path / "autotune.json")
    monkeypatch.delenv("TENSORJIT_RETUNE", raising=False)
    assert store.get(key) == table[key]
    monkeypatch.setenv("TENSORJIT_RETUNE", "1")
    assert store.get(key) is None
    monkeypatch.delenv("TENSORJIT_RETUNE")
    mine = MatmulConfig(64, 64, 16, 4, 2, 2, 32, 1).as_dict()
    store.put(key, mine, 9.0)                      # the user's own measurement wins
    assert store.get(key)["config"] == mine
    assert cache.packaged_entry("no-bars-in-this-key") is None
    assert cache.packaged_entry("hip|gfx000|matmul|x") is None


def test_writers_merge_instead_of_overwriting(tmp_path):
    """Two stores (as two processes would) writing different keys keep both entries, and
    a store sees entries another one wrote after it was opened."""
    path = tmp_path / "autotune.json"
    a, b = cache.AutotuneStore(path), cache.AutotuneStore(path)
    cfg = MatmulConfig(64, 64, 16, 4, 2, 2, 32, 1).as_dict()
    assert a.get("k1") is None and b.get("k2") is None       # both have read the (empty) file
    a.put("k1", cfg, 1.0)
    b.put("k2", cfg, 2.0)
    on_disk = json.loads(path.read_text())
    assert set(on_disk) == {"k1", "k2"}
    assert a.get("k2") == {"config": cfg, "ms": 2.0}
    a.clear()
    assert b.get("k1") is None and not path.exists()


def test_relative_store_name_lives_in_the_cache_dir(tmp_path, monkeypatch):
    monkeypatch.setenv("TENSORJIT_CACHE_DIR", str(tmp_path / "c"))
    assert cache.AutotuneStore().path == tmp_path / "c" / "autotune.json"
    assert cache.AutotuneStore("other.json").path == tmp_path / "c" / "other.json"


def test_code_object_key_covers_source_options_target_and_toolchain(tmp_path, monkeypatch):
    monkeypatch.setenv("TENSORJIT_CACHE_DIR", str(tmp_path))
    base = cache.CodeObjectCache("gfx950:sramecc+:xnack-", "hiprtc7.2-hip70226015")
    opts = ("--offload-arch=gfx950", "-O3")
    base.put("src", opts, b"code")
    assert base.get("src", opts) == b"code"
    misses = [
        cache.CodeObjectCache("gfx950:sramecc+:xnack-", "hiprtc7.3-hip70300000").get("src", opts),  # new compiler
        cache.CodeObjectCache("gfx950:sramecc-:xnack-", "hiprtc7.2-hip70226015").get("src", opts),  # other features
        base.get("src2", opts),
        base.get("src", ("--offload-arch=gfx950", "-O2")),
    ]
    assert misses == [None] * 4
    assert cache.content_hash("ab", "c") != cache.content_hash("a", "bc")


def test_hip_backend_tags_code_objects_with_the_hiprtc_version():
    from tensorjit.backends import hip_backend
    from tensorjit.runtime import hip as rt

    major, minor, runtime = rt.toolchain_version()
    assert major >= 6 and runtime > 0
    tag = hip_backend.toolchain_tag()
    assert f"hiprtc{major}.{minor}" in tag and f"hip{runtime}" in tag


@pytest.mark.parametrize("key", sorted(json.loads((cache.TUNED_DIR / "gfx950.json").read_text())))
def test_every_packaged_config_is_legal_for_its_dtype(key):
    entry = json.loads((cache.TUNED_DIR / "gfx950.json").read_text())[key]
    cfg = MatmulConfig.from_dict(entry["config"])
    assert hip_gemm.config_ok(cfg, DType(key.split("|")[4])), (key, cfg)
    assert entry["ms"] > 0


def test_autotune_times_the_cost_models_best_candidates(tmp_path):
    """The candidates that get timed are the top-k of the hip cost model for the
    (M, N, K, batch) shape, and the fastest measured one is stored."""
    from tensorjit.runtime.autotune import HIP_F32_CANDIDATES, autotune, cost_model

    shape = (512, 768, 3072, 1)
    timed = []

    def build(cfg):
        return cfg

    def timer(cfg, warmup, iters):
        timed.append(cfg)
        return 1.0 + 0.01 * len(timed) if cfg.TM == 64 and cfg.TN == 64 else 5.0

    store = cache.AutotuneStore(tmp_path / "autotune.json")
    best = autotune("k", HIP_F32_CANDIDATES, build, shape, "hip_f32", top_k=3, store=store, timer=timer)
    expect = sorted(HIP_F32_CANDIDATES, key=lambda c: cost_model(c, 512, 768, 3072, "hip_f32", 1))[:3]
    assert set(timed) == set(expect)
    assert store.get("k")["config"] == best.as_dict()
