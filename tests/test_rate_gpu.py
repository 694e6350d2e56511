"""The rate-network engine (MFMA) against the reference's rate fixtures and the oracle.

With float32 storage (``v_mfma_f32_32x32x2_f32``): the free run and every lockstep window
within 1e-4 of each variable's range (the reference's own GPU criterion,
``tests/test_rate.py:30``), gradients within 1e-4 of each gradient's scale. With
bfloat16 storage (``v_mfma_f32_32x32x16_bf16``, rates and weights rounded to 8-bit
mantissas, float32 accumulation) the rates stay within 2e-2 of their range of the float32
oracle's: the rounding of the products, not an error of the step.
"""

import numpy as np
import pytest
import torch

import oracle.rate as oracle_rate
import scenarios as sc
from wiretorch_amd import rate_engine

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAMES = list(sc.RATE_SCENARIOS)


def build(name, device=DEV, **kwargs):
    built = sc.RATE_SCENARIOS[name].build(sc.BATCH_SIZE) if not kwargs else \
        sc.rate_recurrent(sc.BATCH_SIZE, sc.SEED, **kwargs)
    built.model.to(device)
    return built


@pytest.mark.parametrize("name", NAMES)
def test_free_run_on_gpu(name):
    recorded, _ = sc.load_fixture(name)
    record = sc.free_run(sc.RATE_SCENARIOS[name], build(name), device=DEV)
    for key in ("rates", "voltages"):
        atol = 1e-4 * np.ptp(recorded[key])
        np.testing.assert_allclose(record[key], recorded[key], rtol=0, atol=atol, err_msg=key)


@pytest.mark.parametrize("name", NAMES)
def test_lockstep_on_gpu(name):
    scenario = sc.RATE_SCENARIOS[name]
    recorded, _ = sc.load_fixture(name)
    built = build(name)
    model = built.model
    model.track_variables, model.track_batch_idx = True, None
    x = torch.from_numpy(built.input_spikes).to(DEV)
    for w, start in enumerate(range(0, x.shape[1], sc.WINDOW)):
        stop = start + sc.WINDOW
        model.load_checkpoint_state({k: recorded[f"state.{k}"][w] for k in scenario.state_keys})
        with torch.no_grad():
            out = model(x[:, start:stop])
        for key in ("rates", "voltages"):
            atol = 1e-4 * np.ptp(recorded[key])
            np.testing.assert_allclose(out[key].cpu().numpy(), recorded[key][:, start:stop],
                                       rtol=0, atol=atol, err_msg=f"{key}, window {w}")
        for key, value in model.get_checkpoint_state().items():
            ref = recorded[f"state.{key}"][w + 1]
            np.testing.assert_allclose(value, ref, rtol=0, atol=1e-4 * (np.ptp(ref) or 1.0),
                                       err_msg=f"state {key}, window {w}")


@pytest.mark.parametrize("name", NAMES)
def test_gradients_on_gpu(name):
    recorded, _ = sc.load_fixture(name)
    loss, grads = sc.gradients(build(name), device=DEV)
    expected = {k[len("grad."):]: v for k, v in recorded.items() if k.startswith("grad.")}
    assert grads.keys() == expected.keys()
    np.testing.assert_allclose(loss, recorded["loss"], rtol=1e-4)
    for key, value in expected.items():
        scale = np.abs(value).max() or 1.0
        np.testing.assert_allclose(grads[key], value, rtol=0, atol=1e-4 * scale, err_msg=key)


def test_learnt_recurrent_weights_on_gpu():
    """Recurrent weights trained directly (full rank): the engine's plain-product weight
    gradient against the oracle's autograd."""
    results = {}
    for device, engine in (("cpu", oracle_rate), (DEV, None)):
        built = sc.rate_recurrent(sc.BATCH_SIZE, sc.SEED, learnt_excitatory=True)
        built.model.to(device)
        if engine is not None:
            sc.use_engine(built.model, engine)
        results[device] = sc.gradients(built, device=device)
    (l_cpu, g_cpu), (l_gpu, g_gpu) = results["cpu"], results[DEV]
    np.testing.assert_allclose(l_gpu, l_cpu, rtol=1e-4)
    assert g_cpu.keys() == g_gpu.keys()
    for key, value in g_cpu.items():
        scale = np.abs(value).max() or 1.0
        np.testing.assert_allclose(g_gpu[key], value, rtol=0, atol=1e-4 * scale, err_msg=key)


def test_bfloat16_storage_close_to_float32():
    built = sc.rate_recurrent(sc.BATCH_SIZE, sc.SEED, storage_dtype=torch.bfloat16)
    built.model.to(DEV)
    x = torch.from_numpy(built.input_spikes)
    with torch.no_grad():
        r_bf16 = built.model(x.to(DEV)).cpu().numpy()
    ref = sc.rate_recurrent(sc.BATCH_SIZE, sc.SEED)
    sc.use_engine(ref.model, oracle_rate)
    with torch.no_grad():
        r_ref = ref.model(x).numpy()
    np.testing.assert_allclose(r_bf16, r_ref, rtol=0, atol=2e-2 * np.ptp(r_ref))


# ---------------------------------------------------------------------------------
# Dense signed rate network (configuration 4's shape), bfloat16 products
# ---------------------------------------------------------------------------------


def _dense_run(device, engine, **shape):
    """Rates and gradients of a read-out loss, with every product's operands in bfloat16
    (the oracle rounds them the same way and multiplies in float32)."""
    from wiretorch_amd import synthetic

    wl = synthetic.dense_rate(**shape)
    model = wl.model.to(device)
    if engine is not None:
        sc.use_engine(model, engine)
    x = torch.from_numpy(wl.x).to(device)
    g = torch.Generator().manual_seed(11)
    readout = (torch.randn((wl.N, 8), generator=g) / wl.N**0.5).to(device)
    rates = model(x)
    loss = ((rates @ readout) ** 2).mean()
    loss.backward()
    grads = {k: p.grad.detach().cpu().numpy() for k, p in model.named_parameters()}
    return rates.detach().cpu().numpy(), float(loss.detach()), grads


@pytest.mark.parametrize("shape", [
    dict(N=320, n_in=64, B=40, T=60, seed=7),       # ragged: N, B not multiples of 64
    dict(N=384, n_in=64, B=128, T=60, seed=5),      # split products, two k slices
    dict(N=4096, n_in=64, B=256, T=6, seed=4),      # configuration 4's full width (split, 4)
], ids=["small", "split", "config4_width"])
def test_dense_bfloat16_against_rounded_oracle(shape):
    """Every product of two bfloat16 operands is exact in float32, so the engine and the
    oracle differ only in the order of float32 sums — and in the operands whose bfloat16
    rounding that order flips, each moving its terms by 2^-9 of themselves. Those flips
    compound along a chaotic trajectory (g^2 = 1.5): two CPU runs of the oracle that
    differ only in the order of the sums drift apart to 3e-4 of the rates' range by step
    60 (gradients 1e-4 of their scale). So: the first 15 steps within 1e-4 of the range,
    every step within 2e-3 of it, gradients within 1e-3 of their scale."""
    r_ref, l_ref, g_ref = _dense_run("cpu", oracle_rate, **shape)
    r_gpu, l_gpu, g_gpu = _dense_run(DEV, None, **shape)
    ptp = np.ptp(r_ref)
    np.testing.assert_allclose(r_gpu[:, :15], r_ref[:, :15], rtol=0, atol=1e-4 * ptp)
    np.testing.assert_allclose(r_gpu, r_ref, rtol=0, atol=2e-3 * ptp)
    np.testing.assert_allclose(l_gpu, l_ref, rtol=1e-4)
    assert g_ref.keys() == g_gpu.keys()
    for key, value in g_ref.items():
        scale = np.abs(value).max()
        np.testing.assert_allclose(g_gpu[key], value, rtol=0, atol=1e-3 * scale, err_msg=key)


@pytest.mark.parametrize("n", [8, 1000, 4103])
def test_split_bf16_matches_torch_rounding(n):
    """``wt_split_bf16``: hi = bf16(x) and lo = bf16(x - hi), round to nearest even, bit
    for bit as torch's conversions (the vector body and the tail)."""
    from wiretorch_amd.rate_engine import _split
    x = torch.randn(n, device=DEV) * torch.logspace(-6, 6, n, device=DEV)
    hi, lo = _split(x)
    want_hi = x.bfloat16()
    want_lo = (x - want_hi.float()).bfloat16()
    assert torch.equal(hi.view(torch.int16), want_hi.view(torch.int16))
    assert torch.equal(lo.view(torch.int16), want_lo.view(torch.int16))


@pytest.mark.parametrize("K, M, N", [(300, 192, 160), (65_536, 192, 160), (1000, 512, 512),
                                     (4133, 300, 700), (777, 301, 157)])
def test_split_product_error_bound(K, M, N):
    """The weight gradient's product a^T b on the bf16 matrix cores (``wt_gemm_tn_split``:
    operands split in registers into bf16 hi + lo): every entry within 3 * 2^-18 of
    sum |a_i b_i| of the float64 product, on top of float32 accumulation (twice the
    float32 product's own distance to float64: both accumulate in float32, in orders of
    their own), for short and long sums, whole and partial 256 x 256 tiles, a K that is
    no multiple of the 32-step stage and odd widths — no absolute floor."""
    from wiretorch_amd.rate_engine import _gemm_tn
    g = torch.Generator(device=DEV).manual_seed(5)
    a = torch.tanh(torch.randn((K, M), device=DEV, generator=g))
    b = torch.randn((K, N), device=DEV, generator=g) * 1e-3
    exact = a.double().T @ b.double()
    magnitude = a.double().abs().T @ b.double().abs()
    f32 = (a.T @ b).double()
    split = _gemm_tn(a, b).double()
    allowed = 3 * 2.0**-18 * magnitude + 2 * (f32 - exact).abs().max()
    assert bool(((split - exact).abs() <= allowed).all()), float(((split - exact).abs() - allowed).max())
    # strided views (row pitch above the width) give the same result
    wide_a = torch.zeros((K, M + 37), device=DEV)
    wide_a[:, :M] = a
    assert torch.equal(_gemm_tn(wide_a[:, :M], b), _gemm_tn(a, b))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_split_products_match_fused(dtype, monkeypatch):
    """The forward's split product (128 x 128 tiles over k slices, ``wt_rate_split_bytes``)
    against the fused per-step kernel on the same network and input: the same rates and
    gradients up to the order of float32 sums (rates within 1e-5 of their range over 8
    steps, gradients within 1e-4 of their scale). A spy confirms that the split ran."""
    shape = dict(N=384, n_in=64, B=128, T=8, seed=5, storage_dtype=dtype)
    took = []
    real = rate_engine._split_scratch

    def spy(*args):
        out = real(*args)
        took.append(out is not None)
        return out

    monkeypatch.setattr(rate_engine, "_split_scratch", spy)
    r_split, l_split, g_split = _dense_run(DEV, None, **shape)
    assert took and all(took), took
    monkeypatch.setattr(rate_engine, "SPLIT_PRODUCTS", False)
    r_fused, l_fused, g_fused = _dense_run(DEV, None, **shape)
    ptp = np.ptp(r_fused)
    np.testing.assert_allclose(r_split, r_fused, rtol=0, atol=1e-5 * ptp)
    np.testing.assert_allclose(l_split, l_fused, rtol=1e-5)
    for key, value in g_fused.items():
        scale = np.abs(value).max()
        np.testing.assert_allclose(g_split[key], value, rtol=0, atol=1e-4 * scale, err_msg=key)
