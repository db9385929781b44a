"""Host-side behaviour of the LayerAdam drop-in (no GPU needed)."""
from __future__ import annotations

import pytest
import torch

from slideformer_amd import LayerAdam, SUPPORTED_TRIPLES
from slideformer_amd.optimizer import LayerAdam as LayerAdamAlias


def test_import_paths():
    assert LayerAdamAlias is LayerAdam


def test_constructor_defaults_match_reference():
    # layer_adam.py:17-30, 46-53
    adam = LayerAdam()
    assert adam.defaults == dict(lr=1e-3, bias_correction=True, betas=(0.9, 0.999), eps=1e-8,
                                 weight_decay=0, adamw_mode=True)
    assert adam.param_groups == [] and adam.offloader is None and adam.offload_dir is None
    assert adam.fp32_optimizer_state is True and adam.num_layer == 0 and adam.pin_memory is False


def test_stream_shape_options():
    """Keyword-only additions: the chunk and slots host arrays stream with."""
    adam = LayerAdam()
    assert adam.stream_chunk_elems == 16 * 1024 * 1024 and adam.stream_slots == 3
    adam = LayerAdam(stream_chunk_elems=64 * 1024 * 1024, stream_slots=2)
    assert adam.stream_chunk_elems == 64 * 1024 * 1024 and adam.stream_slots == 2
    for bad in (dict(stream_chunk_elems=8), dict(stream_slots=0), dict(stream_slots=17)):
        with pytest.raises(ValueError, match="stream_chunk_elems"):
            LayerAdam(**bad)


def test_unique_optimizer_ids():
    assert LayerAdam().optimizer_id != LayerAdam().optimizer_id


def test_add_layer_params_layout():
    adam = LayerAdam(lr=2e-4, weight_decay=0.01)
    params = [torch.nn.Parameter(torch.randn(3, 4)), torch.nn.Parameter(torch.randn(5))]
    assert adam.add_layer_params(0, params) == 0
    assert adam.add_layer_params(1, []) == -1
    g = adam.param_groups[0]
    assert g["layer_idx"] == 0 and g["step"] == 0 and g["lr"] == 2e-4 and g["params"] == params
    assert adam.exp_avg_flat[0].shape == (17,) and adam.exp_avg_flat[0].dtype == torch.float32
    assert adam.exp_avg_sq_flat[0].abs().sum() == 0
    st = adam.state[params[0]]
    assert st["exp_avg"].shape == (3, 4)
    assert st["exp_avg"].data_ptr() == adam.exp_avg_flat[0].data_ptr()
    assert adam.state[params[1]]["exp_avg_sq"].data_ptr() == adam.exp_avg_sq_flat[0].data_ptr() + 12 * 4


def test_state_dtype_follows_params_when_not_fp32():
    adam = LayerAdam(fp32_optimizer_state=False)
    adam.add_layer_params(0, [torch.nn.Parameter(torch.randn(4).bfloat16())])
    assert adam.exp_avg_flat[0].dtype == torch.bfloat16


def test_begin_chunk_step_and_lr_update():
    adam = LayerAdam()
    adam.add_layer_params(0, [torch.nn.Parameter(torch.randn(4))])
    adam.add_layer_params(1, [torch.nn.Parameter(torch.randn(4))])
    g = adam.begin_chunk_step(1)
    assert g is adam.param_groups[1] and g["step"] == 1 and adam.param_groups[0]["step"] == 0
    adam.end_chunk_step(1)
    adam.update_learning_rate(5e-5)
    assert adam.defaults["lr"] == 5e-5 and all(pg["lr"] == 5e-5 for pg in adam.param_groups)


def test_supported_triples_are_the_references_nine():
    # cpu_adam_impl.cpp:181-189
    assert len(SUPPORTED_TRIPLES) == 9
    assert (torch.float32, torch.bfloat16, torch.float32) in SUPPORTED_TRIPLES
    assert (torch.float32, torch.float32, torch.bfloat16) not in SUPPORTED_TRIPLES


def test_host_tensors_without_gpu_fail_loudly():
    if torch.cuda.is_available():
        pytest.skip("a HIP device is present")
    adam = LayerAdam()
    p = torch.nn.Parameter(torch.randn(8))
    adam.add_layer_params(0, [p])
    p.grad = torch.randn(8)
    with pytest.raises(RuntimeError, match="HIP device"):
        adam.step(0)


def test_moments_device_is_checked_at_construction(tmp_path):
    """moments_device must name a HIP device, and excludes the file offload
    (which moves host-resident moments, layer_adam.py:92-106)."""
    with pytest.raises(ValueError, match="HIP device"):
        LayerAdam(moments_device="cpu")
    with pytest.raises(ValueError, match="exclude each other"):
        LayerAdam(moments_device="cuda:0", nvme_offload_fraction=0.5, offload_dir=str(tmp_path))
    assert LayerAdam(moments_device="cuda:0").moments_device == torch.device("cuda", 0)
    with pytest.raises(ValueError, match="moments_hbm_bytes"):
        LayerAdam(moments_hbm_bytes=1 << 30)
    with pytest.raises(ValueError, match="moments_hbm_bytes"):
        LayerAdam(moments_device="cuda:0", moments_hbm_bytes=-1)


def test_argument_checks_precede_dispatch():
    adam = LayerAdam()
    a = torch.zeros(10)
    with pytest.raises(RuntimeError, match="grads must be contiguous"):
        adam.adam_update(1, 1e-3, 0.9, 0.999, 1e-8, 0, True, a, torch.zeros(10, 2).t()[0], a, a)
    with pytest.raises(RuntimeError, match="size mismatch"):
        adam.adam_update(1, 1e-3, 0.9, 0.999, 1e-8, 0, True, a, a[:3], a, a)
    with pytest.raises(RuntimeError, match="bf16_out"):
        adam.adam_update(1, 1e-3, 0.9, 0.999, 1e-8, 0, True, a, a, a, a, bf16_out=torch.zeros(10))
    with pytest.raises(RuntimeError, match="unsupported device type: meta"):
        adam.adam_update(1, 1e-3, 0.9, 0.999, 1e-8, 0, True, a, a, a.to("meta"), a)


@pytest.mark.parametrize("backend", ["uring", "pthread"])
def test_disk_offloader_round_trip(backend, tmp_path):
    """Native file offload (la_disk_*), the contract LayerAdam uses
    (layer_adam.py:200-247): write, release, read back bit-identical; with
    direct I/O ('uring', the reference's backend) and buffered I/O."""
    from slideformer_amd.nvme import DiskOffloader
    off = DiskOffloader(str(tmp_path), 4, backend)
    assert off.direct == (backend == 'uring')
    a = torch.randn(17 * (1 << 20) + 7)         # 68 MB: two 64 MiB I/O pieces
    b = torch.arange(1000, dtype=torch.float32)
    a_copy, b_copy = a.clone(), b.clone()
    off.async_write(a)
    off.async_write(b)
    off.sync_write_events()
    assert a.untyped_storage().nbytes() == 0 and b.untyped_storage().nbytes() == 0
    assert len(list(tmp_path.glob("offload-*"))) == 2
    off.async_read(a)
    off.async_read(b)
    off.sync_read_events()
    assert torch.equal(a, a_copy) and torch.equal(b, b_copy)
    # a read of a buffer whose release is still pending keeps the in-memory bytes
    b.add_(1)
    off.async_write(b)
    off.async_read(b)
    off.sync_write_events()
    assert torch.equal(b, b_copy + 1)
    del off
    assert list(tmp_path.glob("offload-*")) == []


def test_disk_offloader_never_overlaps_two_writes_of_one_buffer(tmp_path):
    """The reference's prefetch=False hooks (layer_adam.py:226-247) read a layer
    back while its last write is unfenced, step it and write it again.  The
    first write must be fenced before the second is queued (else an old piece
    can land last); the bytes read back after a fenced release are the newest."""
    from slideformer_amd.nvme import DiskOffloader
    off = DiskOffloader(str(tmp_path), 4)
    calls = []

    class Recorder:
        def __init__(self, lib):
            self._lib = lib

        def __getattr__(self, name):
            fn = getattr(self._lib, name)

            def wrapped(*args):
                calls.append(name)
                return fn(*args)
            return wrapped

    off.lib = Recorder(off.lib)
    m = torch.randn(3 * (1 << 20))
    off.async_write(m)          # _post_step: offload
    off.async_read(m)           # next _pre_step: release cancelled, write still queued
    m.mul_(0.5)                 # the step
    off.async_write(m)          # _post_step again
    assert calls == ["la_disk_write_async", "la_disk_sync_writes", "la_disk_write_async"]
    newest = m.clone()
    off.sync_write_events()
    assert m.untyped_storage().nbytes() == 0
    off.async_read(m)
    off.sync_read_events()
    assert torch.equal(m, newest)
    # fenced writes need no extra fence
    calls.clear()
    off.async_write(m)
    off.sync_write_events()
    off.async_read(m)
    off.sync_read_events()
    off.async_write(m)
    assert calls == ["la_disk_write_async", "la_disk_sync_writes", "la_disk_read_async", "la_disk_sync_reads",
                     "la_disk_write_async"]
    off.sync_write_events()
    del off


def test_disk_offloader_errors(tmp_path):
    from slideformer_amd.nvme import DiskOffloader
    not_a_dir = tmp_path / "plain_file"
    not_a_dir.write_bytes(b"x")
    with pytest.raises(OSError):
        DiskOffloader(str(not_a_dir))
    off = DiskOffloader(str(tmp_path))
    with pytest.raises(RuntimeError, match="contiguous"):
        off.async_write(torch.zeros(4, 4).t())
    with pytest.raises(RuntimeError, match="whole"):
        off.async_write(torch.zeros(8)[2:])


def test_layer_adam_nvme_layout_and_offload(tmp_path):
    """nvme_offload_fraction > 0 builds the native offloader; registering
    layers releases the moments of all but the last one (layer_adam.py:191-196)."""
    adam = LayerAdam(nvme_offload_fraction=1.0, offload_dir=str(tmp_path), num_layer=3)
    ps = [torch.nn.Parameter(torch.randn(1000)) for _ in range(3)]
    for i, p in enumerate(ps):
        adam.add_layer_params(i, [p])
    for i in range(2):
        assert adam.exp_avg_flat[i].untyped_storage().nbytes() == 0
        assert adam.exp_avg_sq_flat[i].untyped_storage().nbytes() == 0
    assert adam.exp_avg_flat[2].untyped_storage().nbytes() == 4000
    adam._load_layer(1)
    adam.offloader.sync_read_events()
    assert torch.equal(adam.exp_avg_flat[1], torch.zeros(1000))
    half = LayerAdam(nvme_offload_fraction=0.5, offload_dir=str(tmp_path), num_layer=2)
    half.add_layer_params(0, [torch.nn.Parameter(torch.randn(10))])
    half.add_layer_params(1, [torch.nn.Parameter(torch.randn(10))])
    assert half.exp_avg_flat[0].untyped_storage().nbytes() == 0
    assert half.exp_avg_sq_flat[0].untyped_storage().nbytes() == 40  # only exp_avg below 0.5+


def test_torch_adam_update_formula():
    # the reference's unused pure-torch path, layer_adam.py:250-268
    adam = LayerAdam(weight_decay=0.1)
    data = torch.ones(4)
    grad = torch.full((4,), 0.5)
    m, v = torch.zeros(4), torch.zeros(4)
    adam.torch_adam_update(data, grad, m, v, 0.1, 0.9, 0.999, 1e-8, 0.1, 1 - 0.9, 1 - 0.999)
    expected = 1.0 * (1 - 0.1 * 0.1) - 0.1 * 1.0
    torch.testing.assert_close(data, torch.full((4,), expected), rtol=1e-5, atol=1e-6)


def test_offload_cleanup_leaves_other_processes_files(tmp_path):
    """Tearing LayerAdam down removes this process's offload files and no
    other process's (the reference removes every "offload-*" file of the
    directory, layer_adam.py:117-124)."""
    import gc
    import os

    foreign = tmp_path / "offload-999999999-7"
    foreign.write_bytes(b"another run's moments")
    adam = LayerAdam(nvme_offload_fraction=1.0, offload_dir=str(tmp_path), num_layer=2)
    for i in range(2):
        adam.add_layer_params(i, [torch.nn.Parameter(torch.randn(100))])
    adam.offloader.sync_write_events()
    assert list(tmp_path.glob(f"offload-{os.getpid()}-*"))
    del adam
    gc.collect()
    assert list(tmp_path.glob(f"offload-{os.getpid()}-*")) == []
    assert foreign.read_bytes() == b"another run's moments"


def test_is_page_locked_of_plain_host_memory():
    from slideformer_amd import _lib
    assert not _lib.is_page_locked(torch.zeros(16))
    assert not _lib.is_page_locked(torch.zeros(16)[4:])


def test_disk_offloader_backends_and_direct_fallback(tmp_path, monkeypatch):
    """backend names: 'uring' / 'aio' / 'direct' ask for O_DIRECT, 'pthread' /
    'buffered' for the page cache, anything else is refused.  A file system
    that refuses O_DIRECT (-EINVAL at create) falls back to buffered I/O with a
    warning, and the offload still round-trips."""
    import errno

    from slideformer_amd import _lib
    from slideformer_amd.nvme import DiskOffloader
    with pytest.raises(ValueError, match="unknown backend"):
        DiskOffloader(str(tmp_path), 2, 'io_uring_sqpoll')
    assert DiskOffloader(str(tmp_path), 2, 'aio').direct and not DiskOffloader(str(tmp_path), 2, 'buffered').direct

    real = _lib.load()

    class RefusesDirect:
        def __getattr__(self, name):
            return getattr(real, name)

        def la_disk_create_ex(self, d, threads, flags, out):
            if flags & _lib.LA_DISK_DIRECT:
                return -errno.EINVAL
            return real.la_disk_create_ex(d, threads, flags, out)

    monkeypatch.setattr(_lib, "load", lambda path=None: RefusesDirect())
    with pytest.warns(RuntimeWarning, match="O_DIRECT"):
        off = DiskOffloader(str(tmp_path), 2, 'uring')
    assert not off.direct
    a = torch.arange(5003, dtype=torch.float32)
    ref = a.clone()
    off.async_write(a)
    off.sync_write_events()
    off.async_read(a)
    off.sync_read_events()
    assert torch.equal(a, ref)
    del off


def test_disk_offloader_direct_mode_odd_sizes_and_alignments(tmp_path):
    """Direct I/O with host tensors of sizes that are not whole blocks (the
    bounce buffer and the zero-padded last block; the block-aligned path is
    driven by tests/native/disk_offload_driver.cpp): every byte comes back."""
    from slideformer_amd.nvme import DiskOffloader
    off = DiskOffloader(str(tmp_path), 4, 'direct')
    assert off.direct
    tensors = [torch.randn(k) for k in (1, 3, 1023, 4 * (1 << 20) + 1, 5 * (1 << 20) + 777)]
    tensors.append(torch.randint(0, 255, (4097,), dtype=torch.uint8))
    refs = [t.clone() for t in tensors]
    for t in tensors:
        off.async_write(t)
    off.sync_write_events()
    for t in tensors:
        off.async_read(t)
    off.sync_read_events()
    for t, r in zip(tensors, refs):
        assert torch.equal(t, r)

