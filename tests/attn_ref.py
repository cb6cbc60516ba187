"""Shared fp32 restatement of the absorbed attention for the tests (the
oracle's statement, oracle/latent_ops.absorbed_attention_f64, in fp32 and
row by row so it runs at the BASELINE configurations' sizes; pinned to the
fp64 one, output and log-sum-exp, in tests/test_attn_ref.py).  Reference:
models/mla.py:417-487."""
import torch

H = 16
SCALE = 192 ** -0.5


def ref_attention_fp32(q_abs, q_pe_rot, c_rows, p_rows, lens, scale=SCALE, rank=None):
    """Per row r: s = scale (q_abs.c + q_pe.k_pe) over positions [0, lens[r]),
    o = softmax(s) . c and lse = logsumexp(s) (natural log), in fp32 on the
    inputs' device.  c_rows / p_rows: callables giving row r's fp32 latent /
    rope cache rows [L, R] / [L, P].  Returns (o [rows, H, R], lse [rows, H])."""
    R = q_abs.shape[-1] if rank is None else rank
    rows = q_abs.shape[0]
    out = torch.zeros(rows, H, R, dtype=torch.float32, device=q_abs.device)
    lse = torch.full((rows, H), float("-inf"), dtype=torch.float32, device=q_abs.device)
    for r in range(rows):
        L = int(lens[r])
        if L == 0:
            continue
        c, p = c_rows(r, L), p_rows(r, L)
        s = (q_abs[r, :, :R].float() @ c[:, :R].T + q_pe_rot[r].float() @ p.T) * scale  # [H, L]
        out[r] = torch.softmax(s, dim=-1) @ c[:, :R]
        lse[r] = torch.logsumexp(s, dim=-1)
    return out, lse


def check(out, ref, rtol=2e-2, atol=1e-2):
    """The north-star bf16 attention tolerance."""
    out, ref = out.float(), ref.float()
    err = (out - ref).abs()
    lim = atol + rtol * ref.abs()
    bad = err > lim
    assert not bool(bad.any()), f"{int(bad.sum())}/{bad.numel()} outside tol; max err {float(err.max()):.3e}"


# log-sum-exp bar: one 64-token tile of a 131073-token row moves it by 4.9e-4
LSE_ATOL = 1e-4


def check_lse(lse, ref, atol=LSE_ATOL):
    lse, ref = lse.double().cpu(), ref.double().cpu()
    both_inf = torch.isinf(lse) & torch.isinf(ref) & (lse.sign() == ref.sign())
    err = torch.where(both_inf, torch.zeros_like(lse), (lse - ref).abs())
    assert not bool(torch.isnan(err).any()), "NaN log-sum-exp"
    assert float(err.max()) <= atol, f"log-sum-exp off by {float(err.max()):.3e} (> {atol})"
