"""``wt_cond_run_noalloc`` (the forward whose workspace is the library's own device array)
against ``wt_cond_run`` (the caller's workspace), through the C-ABI: two calls in a row,
the second with a smaller input, each bit-equal to the entry point it stands in for —
spikes, and the state it leaves (v, g, refractory counters) — and the run's error flags
zero. A call whose workspace would exceed the array is refused before anything is
launched."""

import numpy as np
import pytest
import torch

from wiretorch_amd import _lib, engine, synthetic

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(wl, B, T):
    model = wl.model.to(DEV)
    model.reset_state(batch_size=B)
    x = torch.from_numpy(wl.x[:B, :T]).float().to(DEV)
    return model, x


def _run(model, x, entry):
    """One forward of ``model`` over ``x`` through ``entry`` (``"wt_cond_run"`` or
    ``"wt_cond_run_noalloc"``): spikes and final state, as host arrays, and the flags."""
    drive, p = model._drive(), model._physiology()
    L = engine._plan(model.v, x, drive, p, False, False, None)
    B, T, N, S = L.B, L.T, L.N, L.S
    v = model.v.detach().clone()
    # a copy: the permuted view of the network's state may already be contiguous storage
    g = model._synaptic.detach().permute(0, 2, 3, 1).clone(memory_format=torch.contiguous_format)
    counter = model.refractory.detach().clone()
    spikes = torch.full((B, T, N), -1.0, device=DEV)
    groups, R, range_n = L.geo
    geo = L.abi_geometry()
    io = _lib.RunIO(x.data_ptr(), B, T, L.n_in, v.data_ptr(), g.data_ptr(),
                    counter.data_ptr() if L.refractory else None, spikes.data_ptr(),
                    None, None, None, None, None, None, None, None, 0)
    scale = drive.scale.detach().float().contiguous()
    tab, rec, ff = L.abi_tables(scale), L.rec.abi(R, range_n, L.stream), L.ff.abi(R, range_n, L.stream)
    lib = _lib.load()
    flags = torch.full((1,), 0x7fffffff, dtype=torch.int32, device=DEV)
    if entry == "wt_cond_run":
        work = torch.empty(int(lib.wt_cond_run_scratch_bytes(geo, B, T)), dtype=torch.uint8,
                           device=DEV)
        work[: int(lib.wt_cond_run_scratch_zeroed(geo))].zero_()
        _lib.check(lib.wt_cond_run(tab, rec, ff, geo, io, work.data_ptr(), L.stream), entry)
        flags.copy_(work[:4].view(torch.int32))
    else:
        _lib.check(lib.wt_cond_run_noalloc(tab, rec, ff, geo, io, flags.data_ptr(), L.stream),
                   entry)
    torch.cuda.synchronize()
    return [t.cpu().numpy() for t in (spikes, v, g, counter)], int(flags.item())


def test_noalloc_matches_wt_cond_run_on_two_calls():
    wl = synthetic.config1(T=300, B=6)
    for B, T in ((6, 300), (3, 120)):  # the second call smaller than the first
        model, x = _inputs(wl, B, T)
        print(f"noalloc: config1 N={wl.N} B={B} T={T}", flush=True)
        want, want_flags = _run(model, x, "wt_cond_run")
        got, got_flags = _run(model, x, "wt_cond_run_noalloc")
        assert want_flags == 0 and got_flags == 0, (want_flags, got_flags)
        assert want[0].sum() > 0, "no spikes: the check would be vacuous"
        for name, a, b in zip(("spikes", "v", "g", "counter"), got, want):
            np.testing.assert_array_equal(a, b, err_msg=f"{name} (B={B}, T={T})")


def test_noalloc_refuses_a_workspace_beyond_its_array():
    wl = synthetic.config1(T=40, B=2)
    model, x = _inputs(wl, 2, 40)
    L = engine._plan(model.v, x, model._drive(), model._physiology(), False, False, None)
    groups, R, range_n = L.geo
    geo = L.abi_geometry()
    lib = _lib.load()
    T_big = 1_000_000  # input lists alone: 2 * 1e6 * 516 bytes, past the array
    assert lib.wt_cond_run_scratch_bytes(geo, 2, T_big) > _lib.NOALLOC_SCRATCH_BYTES
    io = _lib.RunIO(x.data_ptr(), 2, T_big, L.n_in, 1, 1, None, 1, None, None, None, None,
                    None, None, None, None, 0)  # never dereferenced: refused first
    tab = L.abi_tables(model._drive().scale.detach().float().contiguous())
    rec, ff = L.rec.abi(R, range_n, L.stream), L.ff.abi(R, range_n, L.stream)
    status = lib.wt_cond_run_noalloc(tab, rec, ff, geo, io, None, L.stream)
    assert status == 2  # hipErrorOutOfMemory
