"""Shared tolerances and comparison helpers for the parity tests."""
import torch

# bf16 outputs vs an fp32 oracle computed from the same bf16 inputs.
BF16_ATOL = 2e-2
# fp16 outputs (one ulp at |y| in [1, 2) is 9.8e-4).
F16_ATOL = 1e-2
# fp32 outputs.
F32_ATOL = 1e-4
# logsumexp: |d| <= 1e-3 * max(1, |ref|).
LSE_RTOL = 1e-3

ATOL = {torch.bfloat16: BF16_ATOL, torch.float16: F16_ATOL, torch.float32: F32_ATOL}


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return (a.detach().float().cpu() - b.detach().float().cpu()).abs().max().item()


# Relative term for elementwise outputs whose magnitude exceeds 1 (one bf16
# ulp is 2^-7 relative): |out - ref| <= atol + rtol * |ref|.
RTOL = {torch.bfloat16: 2 ** -7, torch.float16: 2 ** -10, torch.float32: 1e-5}


def assert_close(out: torch.Tensor, ref: torch.Tensor, atol: float, what: str = "",
                 rtol: float = 0.0) -> None:
    assert out.shape == ref.shape, f"{what} shape {tuple(out.shape)} != {tuple(ref.shape)}"
    o = out.detach().float().cpu()
    r = ref.detach().float().cpu()
    assert (o.isnan() == r.isnan()).all(), f"{what}: NaN pattern differs"
    assert (torch.isinf(o) == torch.isinf(r)).all(), f"{what}: inf pattern differs"
    if not o.numel():
        return
    fin = torch.isfinite(r)
    excess = ((o - r).abs() - rtol * r.abs())[fin]
    err = excess.max().item() if excess.numel() else 0.0
    assert err <= atol, f"{what} max abs err beyond rtol {err:.3e} > {atol:.1e}"


def assert_lse_close(out: torch.Tensor, ref: torch.Tensor, what: str = "lse") -> None:
    o = out.detach().float().cpu()
    r = ref.detach().float().cpu()
    assert o.shape == r.shape
    inf = torch.isinf(r)
    assert (torch.isinf(o) == inf).all(), f"{what}: infinite pattern differs"
    fin = ~inf
    if fin.any():
        err = ((o[fin] - r[fin]).abs() / r[fin].abs().clamp(min=1.0)).max().item()
        assert err <= LSE_RTOL, f"{what} rel err {err:.3e} > {LSE_RTOL:.0e}"


def staircase_qkv(B, Hq, Hkv, Sq, Skv, D, dtype, device, seed, step=6.0):
    """Scores that jump by `step` (natural-log units, ~8.7 in log2 units) at
    every 64-key boundary: q rows ~ ones, k_j ~ t_j * ones with t_j rising in
    steps, plus noise. Every 64-key tile then raises each row's running max by
    more than the kernels' lazy-rescale threshold (2^8), so the rescale of O and
    l runs once per tile instead of never (N(0,1) inputs never trigger it past
    the first tile)."""
    g = torch.Generator().manual_seed(seed)
    unit = D ** -0.5 * D  # q . k * scale = t for q = k / t = ones
    t = step * (torch.arange(Skv) // 64).float() / unit
    q = (torch.ones(B, Hq, Sq, D) + 0.1 * torch.randn(B, Hq, Sq, D, generator=g)).to(dtype)
    k = (t[None, None, :, None] * torch.ones(B, Hkv, Skv, D)
         + 0.3 * torch.randn(B, Hkv, Skv, D, generator=g)).to(dtype)
    v = torch.randn(B, Hkv, Skv, D, generator=g).to(dtype)
    return q.to(device), k.to(device), v.to(device)
