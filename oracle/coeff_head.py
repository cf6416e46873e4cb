"""Oracle: the coefficient head of ``SpectralBias.forward`` in torch ops.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  The product runs the
MLP on fused HIP kernels (``scope_coeff_mlp_fwd`` / ``_bwd`` / ``_wgrad``)
and the rest in the fused head kernels (``scope_coeff_head_fwd`` /
``scope_coeff_head_bwd``); this restates the
reference's steps one tensor op at a time, so autograd gives the reference's
gradients.

Restates ``model/attn_bias.py:379-506``:

* the MLP, SiLU between two linear layers (``:380-398``, ``mlp_forward``);
* the MLP output y = [delta_raw | mu_raw | sigma_raw | pi_logits |
  budget_logits | c_raw] (``:419-431``);
* Δ* = σ(delta_raw)·clamp(Δ*max, 0, L-1) (``:438-440``), μ, σ, π = softmax,
  slope = c_scale·tanh (``:445-451``);
* a_mk = exp(-(log ω_k - μ_m)² / 2σ_m²) normalised with +eps, coefficients
  Σ_m π_m a_mk cos/sin(ω_k Δ*_m), b0 = Σ_k coeff_cos (``:458-471``);
* delta_main = Δ*[argmax π], width (``:476-478``);
* in training the four regularisers (``:480-506``).

Disabled mode returns zeros and uniform π (``:411-417``).

Parity pins (tests/test_host.py): vectors recorded from the reference's own
module (``tests/golden/make_reference_vectors.py``), in eval mode and in
training mode with every regulariser together and alone, including the
gradients of the outputs and of reg_loss with respect to q and the MLP
weights.  Runs on any torch device (the GPU tests compare the fused kernels
with it at sizes the CPU would take minutes over).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def mlp_forward(sb, q: torch.Tensor) -> torch.Tensor:
    """The head's MLP (model/attn_bias.py:380-398): SiLU between two linear
    layers, shared across heads or per head, with the weights cast to q's
    dtype."""
    if sb.detach_q:
        q = q.detach()
    dt = q.dtype
    if sb.share_across_heads:
        fc1, fc2 = sb.mlp[0], sb.mlp[2]
        x = F.silu(F.linear(q, fc1.weight.to(dt), fc1.bias.to(dt)))
        return F.linear(x, fc2.weight.to(dt), fc2.bias.to(dt))
    x = F.silu(torch.einsum("bhld,hkd->bhlk", q, sb.w1.to(dt)) + sb.b1.to(dt)[None, :, None, :])
    return torch.einsum("bhlk,hok->bhlo", x, sb.w2.to(dt)) + sb.b2.to(dt)[None, :, None, :]


def coeff_head_forward(sb, q: torch.Tensor, y: torch.Tensor | None = None) -> tuple[torch.Tensor, ...]:
    """The reference's 12-tuple (model/attn_bias.py:385-401) for q [B,H,L,D]
    from the parameters and schedule buffers of ``sb`` (a
    ``scope_amd.SpectralBias``); ``y`` replaces the MLP's output when given
    (to check the head's arithmetic alone on another MLP's output)."""
    B, H, L, Dh = q.shape
    if H != sb.num_heads:
        raise ValueError(f"expected H={sb.num_heads}, got {H}")
    if Dh != sb.head_dim:
        raise ValueError(f"expected head_dim={sb.head_dim}, got {Dh}")
    device = q.device
    Dt = torch.arange(L, device=device, dtype=torch.float32)
    w = sb.omegas.to(device=device)
    c32 = torch.cos(w[:, None] * Dt[None, :])
    s32 = torch.sin(w[:, None] * Dt[None, :])
    cos_wD, sin_wD, cos_mean, sin_mean = c32.to(torch.bfloat16), s32.to(torch.bfloat16), c32.mean(-1), s32.mean(-1)
    if not sb.enabled:
        z_k = q.new_zeros((B, H, L, sb.K), dtype=torch.float32)
        z_l = q.new_zeros((B, H, L), dtype=torch.float32)
        z_m = q.new_zeros((B, H, L, sb.M), dtype=torch.float32)
        z_pi = q.new_full((B, H, L, sb.M), 1.0 / sb.M, dtype=torch.float32)
        return z_k, z_k, z_l, z_l, z_m, z_pi, z_m, z_l, z_l, cos_wD, sin_wD, q.new_zeros((), dtype=torch.float32)
    y = (mlp_forward(sb, q) if y is None else y).float()
    M, K = sb.M, sb.K
    delta_raw, mu_raw, sigma_raw, pi_logits, budget_logits = (y[..., i * M:(i + 1) * M] for i in range(5))
    delta_cap = torch.clamp(sb._delta_star_max_active.to(device=device, dtype=torch.float32), 0.0, float(L - 1))
    delta_star = torch.sigmoid(delta_raw) * delta_cap
    logw_min, logw_max = sb.logw_min.to(device), sb.logw_max.to(device)
    mu = logw_min + (logw_max - logw_min) * torch.sigmoid(mu_raw)
    sigma = 0.25 + 1.75 * torch.sigmoid(sigma_raw)
    pi = torch.softmax(pi_logits, dim=-1)
    if sb.use_slope:
        slope = sb.c_scale * torch.tanh(y[..., 5 * M:5 * M + 1]).squeeze(-1)
    else:
        slope = q.new_zeros((B, H, L), dtype=torch.float32)
    logw = sb.log_omegas.to(device).view(1, 1, 1, 1, K)
    a_mk = torch.exp(-((logw - mu.unsqueeze(-1)) ** 2) / (2 * (sigma.unsqueeze(-1) ** 2)))
    a_mk = a_mk / (a_mk.sum(dim=-1, keepdim=True) + sb.eps)
    phase = sb.omegas.to(device).view(1, 1, 1, 1, K) * delta_star.unsqueeze(-1)
    pi_e = pi.unsqueeze(-1)
    coeff_cos = (pi_e * a_mk * torch.cos(phase)).sum(dim=3)
    coeff_sin = (pi_e * a_mk * torch.sin(phase)).sum(dim=3)
    b0 = coeff_cos.sum(dim=-1) if sb.subtract_b0 else q.new_zeros((B, H, L), dtype=torch.float32)
    main_idx = pi.argmax(dim=-1)
    delta_main = torch.gather(delta_star, -1, main_idx.unsqueeze(-1)).squeeze(-1)
    width = sb.width_min + (sb.width_max - sb.width_min) * torch.sigmoid(mu.mean(dim=-1))

    z = q.new_zeros((), dtype=torch.float32)
    reg_omega = reg_entropy = reg_delta_edge = reg_zero_mean = z
    if sb.training:  # model/attn_bias.py:485-506
        if sb.lambda_omega > 0:
            reg_omega = sb.lambda_omega * (sb.omega_sq.to(device).view(1, 1, 1, 1, K) * a_mk.square()).sum(-1).mean()
        if sb.lambda_entropy > 0:
            entropy = -(pi * (pi + sb.eps).log()).sum(dim=-1)
            h_floor = float(sb.pi_entropy_floor_frac) * math.log(M)
            if h_floor > 0:
                reg_entropy = sb.lambda_entropy * F.relu(entropy.new_tensor(h_floor) - entropy).mean()
        if sb.lambda_zero_mean > 0:
            mean_b = ((coeff_cos * cos_mean).sum(-1) + (coeff_sin * sin_mean).sum(-1)
                      + slope * (0.5 * float(L - 1)) - b0)
            reg_zero_mean = sb.lambda_zero_mean * mean_b.mean().square()
        if sb.lambda_delta_edge > 0:
            edge_eps = sb._delta_edge_eps_active.to(device=device, dtype=torch.float32)
            u = (delta_star / torch.clamp(delta_cap, min=1.0)).clamp(0.0, 1.0)
            edge = F.relu(edge_eps - u) + F.relu(u - (1.0 - edge_eps))
            reg_delta_edge = sb.lambda_delta_edge * edge.mean()
    reg_loss = reg_omega + reg_entropy + reg_delta_edge + reg_zero_mean
    return (coeff_cos, coeff_sin, slope, b0, delta_star, pi, budget_logits, delta_main, width, cos_wD, sin_wD,
            reg_loss)
