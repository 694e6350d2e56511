"""The rate-network engine on MI355X: ``simulate`` with the contract of the reference's
``rate/engine.py`` (and of ``rate/dynamics.simulate``, ``rate/dynamics.py:109-160``),
running ``wt_rate_forward`` / ``wt_rate_backward`` of ``libwiretorch_amd.so``.

Per call the recurrent pathways' weights are laid out as one zero-padded operand (every
pathway a segment of whole 64-row tiles, and its transpose), cached while the weight
tensors are unchanged; the input pathways' activations ``x[:, :, rows] @ W_k`` are one
product for the whole call, before the steps, as in the reference. ``p.storage_dtype``
selects what the products multiply in: float32 (``v_mfma_f32_32x32x2_f32``) or bfloat16
(``v_mfma_f32_32x32x16_bf16``, and operands rounded to bfloat16 for the input product);
state and accumulation stay float32.

Gradients (``_RateRun``, the counterpart of ``rate/engine.py:336-383``) flow to the
inputs, every pathway's weights and kernel scale, and ``theta``, ``gain``, ``beta`` and
``decay``. The weight and input gradients are plain products of the saved rates (or
inputs) with ``dL/da`` (``torch.matmul``). Not supported (raising
``NotImplementedError``): per-step gradient retention (``retain``), float16 storage, CPU
tensors.
"""

from __future__ import annotations

import torch

from wiretorch_amd import _lib
from wiretorch_amd.engine import _cached, _key
from wiretorch_amd.network import Run

TILE = 64
DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1}
#: What the last differentiable forward tracked (returned with its ``Run``).
_LAST_TRACKED = None
#: When a dict, each launch sequence appends a pair of events recorded on its stream
#: just before and after it, under its name: ``"forward"`` (``wt_rate_forward``, T
#: steps), ``"backward"`` (``wt_rate_backward``) and ``"grad_w"`` (the weight and input
#: gradient products). ``bench.py`` times the kernels with them.
LAUNCH_EVENTS: dict | None = None


class _timed:
    """Records a pair of events around a block into ``LAUNCH_EVENTS[name]``."""

    def __init__(self, name):
        self.name = name

    def __enter__(self):
        if LAUNCH_EVENTS is not None:
            self.start = torch.cuda.Event(enable_timing=True)
            self.start.record()

    def __exit__(self, *exc):
        if LAUNCH_EVENTS is not None and exc[0] is None:
            stop = torch.cuda.Event(enable_timing=True)
            stop.record()
            LAUNCH_EVENTS.setdefault(self.name, []).append((self.start, stop))


def _pad(n: int) -> int:
    return -(-n // TILE) * TILE


class _Operand:
    """The padded recurrent weight operand of one drive and what indexes it."""

    def __init__(self, recurrent, N: int, dtype, device):
        self.N, self.N_pad, self.dtype = N, _pad(N), dtype
        rec_sizes = [_pad(rows.numel()) for rows, _ in recurrent]
        self.K_rec_pad = sum(rec_sizes)
        self.seg = []
        W = torch.zeros((self.K_rec_pad, self.N_pad), device=device)
        self.rpos = torch.full((N,), -1, dtype=torch.int32, device=device)
        self.src_of = torch.full((max(self.K_rec_pad, 1),), -1, dtype=torch.int32, device=device)
        start = 0
        for k, ((rows, Wk), size) in enumerate(zip(recurrent, rec_sizes)):
            n_k = rows.numel()
            W[start:start + n_k, :N] = Wk.detach().float()
            self.rpos[rows.long()] = torch.arange(start, start + n_k, dtype=torch.int32,
                                                  device=device)
            self.src_of[start:start + n_k] = rows.to(torch.int32)
            self.seg.append((start, start + size, k, 0))
            start += size
        if len(self.seg) > 16:
            raise NotImplementedError(f"at most 16 recurrent pathways, got {len(self.seg)}")
        self.W = W.to(dtype).contiguous()
        self.Wt = self.W.T.contiguous()  # the forward product reads W along k

    def abi(self, rin, B_pad: int) -> _lib.RateOperand:
        op = _lib.RateOperand()
        op.W = self.W.data_ptr() if self.K_rec_pad else None
        op.Wt = self.Wt.data_ptr() if self.K_rec_pad else None
        op.rin = _lib.ptr(rin)
        op.rpos = self.rpos.data_ptr()
        op.src_of = self.src_of.data_ptr()
        for g, s in enumerate(self.seg):
            for c in range(4):
                op.seg[g][c] = s[c]
        op.n_seg = len(self.seg)
        op.B_pad, op.N_pad = B_pad, self.N_pad
        op.K_rec_pad = self.K_rec_pad
        op.dtype = DTYPE_CODES[self.dtype]
        return op


def _operand(drive, N: int, dtype, device) -> _Operand:
    tensors = [t for pair in drive.recurrent for t in pair]
    key = ("rate_operand", N, str(dtype), str(device)) + _key(*tensors)
    return _cached(key, tuple(tensors), lambda: _Operand(drive.recurrent, N, dtype, device))


def _columns(t: torch.Tensor, rows: torch.Tensor) -> torch.Tensor:
    """``t[..., rows]`` — ``t`` itself (no copy) when ``rows`` are all of its columns in
    order."""
    n = t.shape[-1]
    if rows.numel() == n and bool((rows == torch.arange(n, device=rows.device)).all()):
        return t
    return t[..., rows]


def _input_activations(L, x) -> torch.Tensor | None:
    """``(K_ff, B, T, N)`` float32: ``x[:, :, rows] @ W_k`` per input pathway, one product
    for the whole call as the reference computes it (``network.py:142-157``); with a
    reduced-precision storage dtype the operands are rounded to it and multiplied in
    float32."""
    if not L.K_ff:
        return None
    B, T, N = L.B, L.T, L.N
    A = torch.empty((L.K_ff, B, T, N), device=L.device)
    for j, (rows, W) in enumerate(L.feedforward):
        xr = _columns(x.detach(), rows).reshape(B * T, -1).float()
        Wr = W.detach().float()
        if L.op.dtype != torch.float32:
            # operands rounded to the storage type: their products are exact on the bf16
            # matrix cores (x^T transposed once so that the product is the kernel's a^T b)
            xr, Wr = xr.to(L.op.dtype).float(), Wr.to(L.op.dtype).float()
            _gemm_tn(xr.t().contiguous(), Wr, out=A[j].view(B * T, N))
        else:  # the reference's float32 product
            torch.matmul(xr, Wr, out=A[j].view(B * T, N))
    return A


class _Plan:
    def __init__(self, v, x, drive, p):
        if not x.is_cuda:
            raise NotImplementedError("the rate engine runs on the GPU (CUDA/HIP tensors)")
        if p.storage_dtype not in DTYPE_CODES:
            raise NotImplementedError(f"storage_dtype {p.storage_dtype} (float32 or bfloat16)")
        if drive.sparse_recurrent is not None or drive.sparse_feedforward is not None:
            raise NotImplementedError("compressed connectomes in a rate network")
        self.device = x.device
        self.B, self.T, self.n_in = x.shape
        self.N = v.shape[1]
        self.S = p.sign.shape[0]
        if self.S > 8:
            raise NotImplementedError(f"at most 8 synapse types, got {self.S}")
        self.K_rec, self.K_ff = len(drive.recurrent), len(drive.feedforward)
        self.K = self.K_rec + self.K_ff
        self.feedforward = drive.feedforward
        self.B_pad = _pad(self.B)
        self.op = _operand(drive, self.N, p.storage_dtype, self.device)
        f = lambda t: t.detach().to(device=self.device, dtype=torch.float32).contiguous()
        self.jump = torch.stack(
            [drive.scale[k][:, None] * drive.made[k] for k in range(self.K)]
        ).detach().float().contiguous() if self.K else torch.zeros((1, self.N, self.S), device=self.device)
        self.made = drive.made.detach().float().contiguous()
        self.theta, self.gain, self.beta = f(p.theta), f(p.gain), f(p.beta)
        self.sign, self.decay = f(p.sign), f(p.decay)
        self.nl = p.nonlinearity.to(device=self.device, dtype=torch.int8).contiguous()

    def tables(self) -> _lib.RateTables:
        return _lib.RateTables(
            self.theta.data_ptr(), self.gain.data_ptr(), self.beta.data_ptr(),
            self.nl.data_ptr(), self.sign.data_ptr(), self.decay.data_ptr(),
            self.jump.data_ptr(), self.made.data_ptr(), self.N, self.S, self.K, self.K_rec,
        )  # fmt: skip


#: Whether the forward's split product (``wt_rate_split_bytes``) may run where it applies;
#: off, every step runs the fused kernel.
SPLIT_PRODUCTS = True


def _split_scratch(tables, op, B: int, device) -> torch.Tensor | None:
    """The split product's scratch, or None where it does not apply."""
    if not SPLIT_PRODUCTS:
        return None
    nbytes = int(_lib.load().wt_rate_split_bytes(tables, op, B))
    return torch.empty(nbytes // 4, device=device) if nbytes else None


def _forward(L: _Plan, x, v, I, track, track_b, saved):
    """One ``wt_rate_forward`` launch sequence; ``v`` ``(B, N)`` and ``I`` ``(B, S, N)`` are
    updated in place. Returns the rates and the tracked variables."""
    B, T, N, S = L.B, L.T, L.N, L.S
    dev = L.device
    out = torch.empty((B, T, N), device=dev)
    Bt = B if track_b < 0 else 1
    tv = torch.empty((Bt, T, N), device=dev) if track else None
    tI = torch.empty((Bt, T, N, S), device=dev) if track else None
    rin = torch.zeros((2, L.B_pad, max(L.op.K_rec_pad, 1)), dtype=L.op.dtype, device=dev)
    A_ff = _input_activations(L, x)
    v_s, I_s, tgt_s, A_s = saved if saved is not None else (None,) * 4
    tables, op = L.tables(), L.op.abi(rin, L.B_pad)
    split = _split_scratch(tables, op, B, dev)
    io = _lib.RateIO(B, T, v.data_ptr(), I.data_ptr(), out.data_ptr(), _lib.ptr(tv),
                     _lib.ptr(tI), track_b, _lib.ptr(v_s), _lib.ptr(I_s), _lib.ptr(tgt_s),
                     _lib.ptr(A_s), _lib.ptr(A_ff), _lib.ptr(split))
    stream = torch.cuda.current_stream(dev).cuda_stream
    with _timed("forward"):
        _lib.check(_lib.load().wt_rate_forward(tables, op, io, stream), "wt_rate_forward")
    tracked = {"v": tv, "I": tI} if track else None
    return out, tracked


class _RateRun(torch.autograd.Function):
    """Rates of a chunk, differentiable in the kernel ``scale``, the input ``x``, the
    pathways' weights, ``theta``, ``gain``, ``beta`` and ``decay``."""

    @staticmethod
    def forward(ctx, L: _Plan, track, track_b, v, I, scale, x, theta, gain, beta, decay, *weights):
        B, T, N, S, K = L.B, L.T, L.N, L.S, L.K
        dev = L.device
        want_decay = decay.requires_grad
        want_scale = scale.requires_grad
        v_s = torch.empty((B, T, N), device=dev)
        I_s = torch.empty((B, T, N, S), device=dev) if (beta.requires_grad or want_decay
                                                       or want_scale) else None
        tgt_s = torch.empty((B, T, N, S), device=dev) if (want_decay or want_scale) else None
        A_s = torch.empty((max(K, 1), B, T, N), device=dev) if want_scale else None
        out, tracked = _forward(L, x, v, I, track, track_b, (v_s, I_s, tgt_s, A_s))
        global _LAST_TRACKED
        _LAST_TRACKED = tracked
        ctx.L = L
        ctx.save_for_backward(out, x, v_s,
                              *(t if t is not None else out.new_empty(0) for t in (I_s, tgt_s, A_s)),
                              I.clone(), *weights)
        ctx.mark_non_differentiable(v, I)
        return out, v, I

    @staticmethod
    def backward(ctx, grad_out, _v, _I):
        L = ctx.L
        out, x, v_s, I_s, tgt_s, A_s, I_final, *weights = ctx.saved_tensors
        needs = ctx.needs_input_grad
        want_scale, want_x = needs[5], needs[6]
        want_theta, want_gain, want_beta, want_decay = needs[7:11]
        w_needs = needs[11:]
        B, T, N, S, K = L.B, L.T, L.N, L.S, L.K
        dev = L.device
        zeros = lambda *shape: torch.zeros(shape, device=dev)
        if grad_out is None:
            grad_out = torch.zeros_like(out)
        grad_A = torch.empty((max(K, 1), B, T, N), device=dev)
        rec = L.K_rec > 0
        gA_op = (torch.zeros((L.K_rec, L.B_pad, L.op.N_pad), dtype=L.op.dtype, device=dev)
                 if rec else None)
        acc = {
            "theta": zeros(B, N) if want_theta else None,
            "gain": zeros(B, N) if want_gain else None,
            "beta": zeros(B, N) if want_beta else None,
            "decay": zeros(B, S, N) if want_decay else None,
            "scale": zeros(max(K, 1), B, N) if want_scale else None,
        }
        # every buffer the launches read or write is held by a name until they are queued
        # (the allocator then reuses memory in stream order only)
        grad_out = grad_out.contiguous()
        lam_v, lam_I = zeros(B, N), zeros(B, S, N)
        d_rate = zeros(B, N) if rec else None
        rin = torch.zeros((2, L.B_pad, max(L.op.K_rec_pad, 1)), dtype=L.op.dtype, device=dev)
        io = _lib.RateBackIO(
            B, T, grad_out.data_ptr(), v_s.data_ptr(),
            I_s.data_ptr() if I_s.numel() else None,
            tgt_s.data_ptr() if tgt_s.numel() else None,
            A_s.data_ptr() if A_s.numel() else None, I_final.data_ptr(),
            lam_v.data_ptr(), lam_I.data_ptr(), _lib.ptr(d_rate), _lib.ptr(gA_op),
            grad_A.data_ptr(),
            *[_lib.ptr(acc[k]) for k in ("theta", "gain", "beta", "decay", "scale")],
        )  # fmt: skip
        stream = torch.cuda.current_stream(dev).cuda_stream
        with _timed("backward"):
            _lib.check(_lib.load().wt_rate_backward(L.tables(), L.op.abi(rin, L.B_pad),
                                                    io, stream), "wt_rate_backward")
        grad_scale = acc["scale"].sum(dim=1)[:K] if want_scale else None
        grad_theta = acc["theta"].sum(0) if want_theta else None
        grad_gain = acc["gain"].sum(0) if want_gain else None
        grad_beta = acc["beta"].sum(0) if want_beta else None
        grad_decay = acc["decay"].sum(dim=(0, 2)) if want_decay else None
        # weights and inputs: plain products with dL/da
        with _timed("grad_w"):
            grad_w, grad_x = _weight_and_input_grads(L, out, x, grad_A, weights, w_needs,
                                                     want_x)
        if grad_x is not None:
            grad_x = grad_x.to(x.dtype)
        return (None, None, None, None, None, grad_scale, grad_x, grad_theta, grad_gain,
                grad_beta, grad_decay, *grad_w)


def _split(x: torch.Tensor):
    """``(hi, lo)`` bfloat16 with ``x = hi + lo`` to 2^-17 relative (``wt_split_bf16``)."""
    x = x.float().contiguous()
    if x.data_ptr() % 16:  # the kernel moves 16-byte vectors
        x = x.clone()
    hi = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    lo = torch.empty_like(hi)
    _lib.check(_lib.load().wt_split_bf16(x.data_ptr(), x.numel(), hi.data_ptr(), lo.data_ptr(),
                                         torch.cuda.current_stream(x.device).cuda_stream),
               "wt_split_bf16")
    return hi, lo


def _gemm_tn(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``a^T b`` of float32 ``(K, M)`` and ``(K, N)`` matrices on the bf16 matrix cores
    (``wt_gemm_tn_split``): each operand split in registers into bf16 hi + lo, the product
    hi.hi + hi.lo + lo.hi accumulated in float32 — every term within 3 * 2^-18 of its
    float32 value (float32's product: 2^-24), before the float32 accumulation both share;
    exact products where both operands are bfloat16 values (lo = 0). ``out``: a
    contiguous float32 ``(M, N)`` to write."""
    a, b = a.float(), b.float()
    if a.stride(1) != 1:
        a = a.contiguous()
    if b.stride(1) != 1:
        b = b.contiguous()
    K, M = a.shape
    N = b.shape[1]
    C = torch.empty((M, N), dtype=torch.float32, device=a.device) if out is None else out
    if C.shape != (M, N) or C.dtype != torch.float32 or not C.is_contiguous():
        raise ValueError("out: a contiguous float32 (M, N) tensor expected")
    _lib.check(_lib.load().wt_gemm_tn_split(
        a.data_ptr(), a.stride(0), b.data_ptr(), b.stride(0), C.data_ptr(), N, K, M, N, 0,
        torch.cuda.current_stream(a.device).cuda_stream), "wt_gemm_tn_split")
    return C


def _weight_and_input_grads(L: _Plan, out, x, grad_A, weights, w_needs, want_x):
    """``dL/dW_k = sum_{b,t} pre ⊗ dL/da_k`` (``pre``: the source rates, or the inputs) and
    ``dL/dx = dL/da_k W_k^T`` per input pathway (``rate/engine.py:367-376``), float32."""
    B, T, N = L.B, L.T, L.N
    grad_w = [None] * len(weights)
    for k, rows in enumerate(L.rows_rec):
        if not w_needs[k]:
            continue
        pre = _columns(out, rows).reshape(B * T, -1)
        g = grad_A[k].reshape(B * T, N)
        if L.op.dtype == torch.float32:  # the reference's precision: its float32 product
            grad_w[k] = pre.T @ g
        else:  # reduced-precision storage: the split product on the bf16 matrix cores
            grad_w[k] = _gemm_tn(pre, g)
    grad_x = torch.zeros_like(x, dtype=torch.float32) if want_x else None
    for j, (rows, W) in enumerate(zip(L.rows_ff, weights[L.K_rec:])):
        k = L.K_rec + j
        g = grad_A[k].reshape(B * T, N)
        if w_needs[k]:
            grad_w[k] = _columns(x.detach().float(), rows).reshape(B * T, -1).T @ g
        if want_x:
            grad_x[:, :, rows] += (g @ W.detach().float().T).reshape(B, T, -1)
    return grad_w, grad_x


def simulate(v, I, x, drive, p, *, probabilities=False, track=False, track_batch_idx=None,
             retain=None) -> Run:
    """Simulate ``x.shape[1]`` steps from ``(v, I)`` (``(B, N)``, ``(B, N, S)``); the
    contract of ``rate/dynamics.py:109-160``."""
    assert not probabilities, "rate networks have no spike probabilities"
    if retain is not None:
        raise NotImplementedError("per-step gradient retention (track_gradients)")
    L = _Plan(v, x, drive, p)
    L.rows_rec = [rows.long() for rows, _ in drive.recurrent]
    L.rows_ff = [rows.long() for rows, _ in drive.feedforward]
    dev = L.device
    v = v.detach().to(device=dev, dtype=torch.float32).clone(memory_format=torch.contiguous_format)
    I_state = I.detach().to(device=dev, dtype=torch.float32).permute(0, 2, 1).clone(
        memory_format=torch.contiguous_format)
    track_b = -1 if track_batch_idx is None else int(track_batch_idx)
    weights = [W for _, W in drive.recurrent] + [W for _, W in drive.feedforward]
    params = (drive.scale, x, p.theta, p.gain, p.beta, p.decay, *weights)
    grad = torch.is_grad_enabled() and any(t.requires_grad for t in params)
    if grad:
        out, v, I_state = _RateRun.apply(L, track, track_b, v, I_state, drive.scale, x,
                                         p.theta, p.gain, p.beta, p.decay, *weights)
        tracked = _LAST_TRACKED if track else None
    else:
        with torch.no_grad():
            out, tracked = _forward(L, x, v, I_state, track, track_b, None)
    return Run(output=out, v=v, syn=I_state.permute(0, 2, 1), tracked=tracked)
