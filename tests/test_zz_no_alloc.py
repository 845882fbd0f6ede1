"""The no-allocation entry point (fh_encode_device_noalloc) against
fh_encode_device: same inputs, same bits, on two calls in a row (the second
smaller, so the scratch holds the first call's leftovers), plus its size
limit.  Called through the C ABI."""
import numpy as np
import pytest

from futon_amd import _lib, synth

pytestmark = pytest.mark.gpu


def _run(L, entry, m, ids, offsets, od):
    import torch
    dev = torch.device("cuda:0")
    d_ids, d_off = torch.from_numpy(ids).to(dev), torch.from_numpy(offsets).to(dev)
    nseq = offsets.size - 1
    d_out = torch.full((nseq, od), float("nan"), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    rc = entry(m.handle, d_ids.data_ptr(), d_off.data_ptr(), nseq, int(offsets[-1]), int(np.diff(offsets).max()),
               0, d_out.data_ptr(), torch.cuda.current_stream().cuda_stream, offsets.ctypes.data)
    _lib.check(rc, "encode")
    torch.cuda.synchronize()
    return d_out.cpu().numpy()


@pytest.mark.parametrize("name", ["bge-small", "nomic-bert", "bge-small-q8"])
def test_noalloc_matches_device_entry(name):
    from futon_amd import native
    L = _lib.load()
    w = synth.workload(name)
    tensors = synth.make_tensors(w.config, w.weight_seed, biases=w.extra.get("biases", True), q8=w.q8)
    m = native.Model(native.PackConfig.from_dict(w.config), tensors, q8=w.q8)
    od = w.config["hidden_size"]
    # nomic: sequences past one key block (multi-block attention), ~3k tokens
    lo, hi, b1, b2 = (16, 128, 24, 9) if name != "nomic-bert" else (129, 400, 10, 4)
    for batch, seed in ((b1, 1), (b2, 2)):  # the second call smaller than the first
        ids, offsets = synth.make_batch(w.ids_seed + seed, batch, lo, hi)
        ids = np.ascontiguousarray(ids)
        offsets = np.ascontiguousarray(offsets)
        want = _run(L, L.fh_encode_device, m, ids, offsets, od)
        got = _run(L, L.fh_encode_device_noalloc, m, ids, offsets, od)
        assert np.isfinite(want).all()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (name, batch)
        print(f"{name}: B={batch} T={int(offsets[-1])} no-alloc == device entry", flush=True)
    m.close()


def test_noalloc_rejects_batches_beyond_its_scratch():
    import torch
    from futon_amd import native
    L = _lib.load()
    assert L.fh_noalloc_scratch_bytes() == 64 << 20
    w = synth.workload("bge-small")
    tensors = synth.make_tensors(w.config, w.weight_seed)
    m = native.Model(native.PackConfig.from_dict(w.config), tensors)
    ids, offsets = synth.make_batch(w.ids_seed, 256, 16, 128)  # 18048 tokens: ~180 MB of workspace
    dev = torch.device("cuda:0")
    d_ids, d_off = torch.from_numpy(ids).to(dev), torch.from_numpy(offsets).to(dev)
    d_out = torch.zeros((256, 384), dtype=torch.float32, device=dev)
    rc = L.fh_encode_device_noalloc(m.handle, d_ids.data_ptr(), d_off.data_ptr(), 256, int(offsets[-1]),
                                    int(np.diff(offsets).max()), 0, d_out.data_ptr(), None, None)
    assert rc == _lib.FH_EINVAL
    assert "scratch" in _lib.last_error()
    torch.cuda.synchronize()
    assert (d_out.cpu().numpy() == 0).all()
    m.close()
