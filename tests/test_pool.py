"""Output pool contract (reference ``tensorjit/runtime/executor.py:19-79`` and its test
``tests/test_backends.py:190-206``): a returned buffer is reused only once the caller
holds nothing that can still see its memory.  CPU tensors here; the GPU executor uses
the same pool (``test_output_buffers_reused_only_when_dropped`` on the GPU)."""
import torch

from tensorjit.runtime.pool import BufferPool

SHAPE, DT, DEV = (64, 32), torch.float32, "cpu"


def take(pool):
    return pool.take_output(SHAPE, DT, DEV)


def test_dropped_output_is_reused_and_has_the_right_layout():
    pool = BufferPool()
    a = take(pool)
    assert a.shape == SHAPE and a.dtype == DT and a.is_contiguous()
    p = a.data_ptr()
    del a
    b = take(pool)
    assert b.data_ptr() == p and pool.held() == 1


def test_anything_the_caller_still_holds_blocks_reuse():
    pool = BufferPool()
    out = take(pool)
    p = out.data_ptr()
    holders = {
        "tensor": lambda t: t,
        "view": lambda t: t[3:],
        "reshape": lambda t: t.reshape(-1),
        "detach": lambda t: t.detach(),
        "storage": lambda t: t.untyped_storage(),
        "numpy": lambda t: t.numpy(),
        # autograd saves the output's TensorImpl (not its Python object) for the backward
        "autograd": lambda t: t * torch.ones(1, requires_grad=True),
    }
    for name, make in holders.items():
        keep = make(out)
        del out
        other = take(pool)
        assert other.data_ptr() != p, name
        del other, keep
        out = take(pool)
        assert out.data_ptr() == p, name      # free again once the holder is gone


def test_values_written_by_the_caller_survive_other_calls():
    pool = BufferPool()
    a = take(pool)
    a.fill_(1.0)
    b = take(pool)
    b.fill_(2.0)
    assert bool((a == 1.0).all()) and a.data_ptr() != b.data_ptr()


def test_at_most_max_held_storages_per_key():
    pool = BufferPool()
    kept = [take(pool) for _ in range(BufferPool.MAX_HELD + 3)]
    assert pool.held() == BufferPool.MAX_HELD
    assert len({t.data_ptr() for t in kept}) == len(kept)
    # a different shape or dtype is a different key
    pool.take_output((4,), DT, DEV)
    pool.take_output(SHAPE, torch.bfloat16, DEV)
    assert pool.held() == BufferPool.MAX_HELD + 2


def test_scalar_outputs():
    pool = BufferPool()
    s = pool.take_output((), DT, DEV)
    assert s.shape == () and s.numel() == 1
    p = s.data_ptr()
    del s
    assert pool.take_output((), DT, DEV).data_ptr() == p
