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
    assert cache._packaged("no-bars-in-this-key") is None
    assert cache._packaged("hip|gfx000|matmul|x") is None


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
