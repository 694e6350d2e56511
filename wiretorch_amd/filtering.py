"""Causal double-exponential filtering of spike trains along time, on MI355X.

``double_exponential`` has the contract of the reference's
``training_utils/filtering.py:28-48``: it filters ``(batch, time, n)`` trains first with
the rise and then with the decay exponential, continuing from carried state,

    rise[t]   = a_r rise[t - 1] + x[t],      rise[-1]   = carried_rise
    smooth[t] = a_d smooth[t - 1] + rise[t], smooth[-1] = carried_smooth

with the carried state entering undecayed at ``t = 0`` (``filtering.py:113-122``). That
is the literal sum ``sum_k a^k x[t - k] + carried a^t`` of the docstring, computed in
linear time. The forward and its reverse recursion run as ``wt_filter_forward`` /
``wt_filter_backward`` of ``libwiretorch_amd.so``, one lane per (trial, neuron) column;
each multiply and add is rounded separately. No gradient flows into the carried states
or through ``rise`` (``filtering.py:84``).

CPU tensors raise: there is no CPU path here.
"""

from __future__ import annotations

import torch

from wiretorch_amd import _lib


def double_exponential(
    x: torch.Tensor,
    kernel_rise: torch.Tensor,
    kernel_decay: torch.Tensor,
    carried_rise: torch.Tensor | None,
    carried_smooth: torch.Tensor | None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Filter ``x`` ``(B, T, N)``; return ``(rise, smooth)``, each ``(B, T, N)`` float32.

    ``kernel_*[k] = exp(-k dt / tau)``: only ``kernel_*[1]``, the one-step decay, is used.
    The carried states are ``(B, 1, N)`` or None (zero). Mirrors
    ``training_utils/filtering.py:28-48``.
    """
    if not x.is_cuda:
        raise RuntimeError(f"the HIP filter runs on a GPU; the input is on {x.device}")
    if x.ndim != 3:
        raise ValueError(f"expected (batch, time, n) trains, got shape {tuple(x.shape)}")
    B, _, N = x.shape
    for name, c in (("carried_rise", carried_rise), ("carried_smooth", carried_smooth)):
        if c is not None and tuple(c.shape) != (B, 1, N):
            raise ValueError(f"{name} must be (B, 1, N) = {(B, 1, N)}, got {tuple(c.shape)}")
    return _DoubleExponential.apply(
        x, _step_decay(kernel_rise), _step_decay(kernel_decay), carried_rise, carried_smooth
    )


def _step_decay(kernel: torch.Tensor) -> float:
    """``kernel[1]`` as a float, read from the device once per kernel tensor
    (``filtering.py:51-61``)."""
    decay = getattr(kernel, "_step_decay", None)
    if decay is None:
        decay = kernel._step_decay = float(kernel[1])
    return decay


def _carried(c, x):
    if c is None:
        return None
    return c.detach().to(device=x.device, dtype=torch.float32).contiguous()


class _DoubleExponential(torch.autograd.Function):
    """Forward and reverse recursion (``filtering.py:75-97``); gradient to ``x`` only."""

    @staticmethod
    def forward(ctx, x, a_rise, a_decay, carried_rise, carried_smooth):
        x = x.float().contiguous()
        B, T, N = x.shape
        rise, smooth = torch.empty_like(x), torch.empty_like(x)
        cr, cs = _carried(carried_rise, x), _carried(carried_smooth, x)
        with torch.cuda.device(x.device):
            stream = torch.cuda.current_stream(x.device).cuda_stream
            _lib.check(_lib.load().wt_filter_forward(
                x.data_ptr(), _lib.ptr(cr), _lib.ptr(cs), rise.data_ptr(), smooth.data_ptr(),
                a_rise, a_decay, B, T, N, stream), "wt_filter_forward")  # fmt: skip
        ctx.shape, ctx.decays = (B, T, N), (a_rise, a_decay)
        ctx.mark_non_differentiable(rise)
        return rise, smooth

    @staticmethod
    def backward(ctx, _grad_rise, grad_smooth):
        B, T, N = ctx.shape
        grad_smooth = grad_smooth.float().contiguous()
        grad_x = torch.empty((B, T, N), device=grad_smooth.device)
        with torch.cuda.device(grad_smooth.device):
            stream = torch.cuda.current_stream(grad_smooth.device).cuda_stream
            _lib.check(_lib.load().wt_filter_backward(
                grad_smooth.data_ptr(), grad_x.data_ptr(), *ctx.decays, B, T, N, stream),
                "wt_filter_backward")  # fmt: skip
        return grad_x, None, None, None, None


class VanRossumLoss(torch.nn.Module):
    """Van Rossum distance between spike trains, with the double-exponential filter.

    Mirrors ``training_utils/losses.py:30-135``: both trains are filtered (rise, then
    decay), carrying the filter state from chunk to chunk with no gradient across chunks,
    and the loss is the mean squared difference of the results. Accepts
    ``(batch, time, n)`` or ``(batch, patterns, time, n)``.
    """

    required_inputs = ["output_spikes", "target_spikes"]
    requires_target = True
    CARRIED_STATE = (
        "prev_output_rise",
        "prev_target_rise",
        "prev_output_smooth",
        "prev_target_smooth",
    )

    def __init__(self, tau_rise: float, tau_decay: float, dt: float, window_size: int,
                 device: str = "cuda", debug: bool = False):  # fmt: skip
        super().__init__()
        self.tau_rise, self.tau_decay, self.dt = tau_rise, tau_decay, dt
        self.kernel_size = window_size
        self.debug = debug
        t = torch.arange(window_size, dtype=torch.float32, device=device) * dt
        self.register_buffer("kernel_rise", torch.exp(-t / tau_rise))
        self.register_buffer("kernel_decay", torch.exp(-t / tau_decay))
        self.reset_state()

    def smooth(self, output_spikes, target_spikes):
        """Filter both trains from (and updating) the carried state; ``(B, T, N)`` each."""
        output_spikes, target_spikes = output_spikes.float(), target_spikes.float()
        if output_spikes.ndim == 4:
            output_spikes, target_spikes = output_spikes.flatten(0, 1), target_spikes.flatten(0, 1)
        kernels = self.kernel_rise, self.kernel_decay
        o_rise, o_smooth = double_exponential(
            output_spikes, *kernels, self.prev_output_rise, self.prev_output_smooth)
        t_rise, t_smooth = double_exponential(
            target_spikes, *kernels, self.prev_target_rise, self.prev_target_smooth)
        self.prev_output_rise = o_rise[:, -1:].detach()
        self.prev_target_rise = t_rise[:, -1:].detach()
        self.prev_output_smooth = o_smooth[:, -1:].detach()
        self.prev_target_smooth = t_smooth[:, -1:].detach()
        return o_smooth, t_smooth

    def forward(self, output_spikes, target_spikes):
        output_smooth, target_smooth = self.smooth(output_spikes, target_spikes)
        loss = ((output_smooth - target_smooth) ** 2).mean()
        if self.debug:
            per_neuron = lambda y: y.permute(0, 2, 1).reshape(-1, 1, y.shape[1])  # noqa: E731
            return loss, per_neuron(output_smooth), per_neuron(target_smooth)
        return loss

    def reset_state(self):
        """Forget the carried filter state (call at the start of a new sequence)."""
        for name in self.CARRIED_STATE:
            setattr(self, name, None)
