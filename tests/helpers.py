"""Shared helpers for the parity tests: seeded inputs, torch <-> numpy bit views, error metric."""
import numpy as np
import torch

from oracle import contract as C

TORCH_CODE = {torch.float32: C.DT_F32, torch.bfloat16: C.DT_BF16, torch.float16: C.DT_F16,
              torch.float64: C.DT_F64}


def normwise(y, ref):
    """max|y - ref| / max|ref| over the whole tensor (the reference's metric,
    tests/test_pallas_afa.py:110-113)."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    return float(np.max(np.abs(y - ref)) / np.max(np.abs(ref)))


def to_bits(t: torch.Tensor) -> np.ndarray:
    """Tensor -> numpy in the C oracle's representation (uint16 bits for bf16/fp16)."""
    t = t.detach().contiguous().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def to_f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().to(torch.float64).numpy()


def from_bits(a: np.ndarray, dtype: torch.dtype, device) -> torch.Tensor:
    if dtype in (torch.bfloat16, torch.float16):
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(dtype).to(device)
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def make_qkv(shape, dtype, seed=0, scale=1.0, device="cuda"):
    """q, k, v ~ scale * N(0,1), drawn in fp64 with numpy's default_rng(seed) in the order q, k, v
    and rounded once to dtype (RNE)."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(3):
        x = rng.standard_normal(shape) * scale
        out.append(torch.from_numpy(x).to(dtype).to(device))
    return out


def oracle_contract(q, k, v, sink=0.5, causal=False, valid_len=None, rotary=None):
    """Run the C contract oracle on the exact input bits of q, k, v."""
    code = TORCH_CODE[q.dtype]
    rot = None
    if rotary is not None:
        tdt = np.float64 if q.dtype == torch.float64 else np.float32
        rot = (rotary[0].detach().cpu().numpy().astype(tdt), rotary[1].detach().cpu().numpy().astype(tdt))
    out, d = C.afa_fwd(to_bits(q), to_bits(k), to_bits(v), code, sink, causal, valid_len, rot)
    return C.to_f32(out, code).astype(np.float64), d.astype(np.float64)


def afa_rows_forward64(q, k, v, rows, sink=0.5):
    """float64 causal AFA forward of the query rows `rows` of one head only (q, k, v: (L, D)
    float64), each row from its own keys 0..i: O(len(rows) L D), so full-length rows stay cheap.
    Returns (out rows, d rows).  Same formula as oracle afa_forward (pinned against it on the CPU)."""
    from oracle import afa_oracle as O

    scale = 1.0 / np.sqrt(q.shape[-1])
    outs, dens = [], []
    for i in rows:
        w = O.rho8((k[: i + 1] @ q[i]) * scale)
        d = w.sum() + sink
        outs.append((w @ v[: i + 1]) / d)
        dens.append(d)
    return np.array(outs), np.array(dens)


def afa_rows_backward64(q, k, v, g, out, den, qrows, krows):
    """float64 causal AFA backward restricted to the dq rows `qrows` and the dk / dv rows `krows`
    of one head, from the given forward residuals (out (L, D), den (L,)) as the reference's
    backward takes them (E_i = g_i . out_i, w_ij = rho8(s_ij) / den_i,
    ds_ij = 8 scale r_ij w_ij (g_i . v_j - E_i); src/kernels/pallas_afa.py:451-517).
    O((len(qrows) + len(krows)) L D).  Pinned against oracle afa_backward on the CPU."""
    from oracle import afa_oracle as O

    scale = 1.0 / np.sqrt(q.shape[-1])
    E = np.sum(g * out, axis=-1)
    dq = []
    for i in qrows:
        s = (k[: i + 1] @ q[i]) * scale
        ds = 8.0 * scale * O.rho8(s) / den[i] / np.sqrt(1.0 + s * s) * (v[: i + 1] @ g[i] - E[i])
        dq.append(ds @ k[: i + 1])
    dk, dv = [], []
    for j in krows:
        s = (q[j:] @ k[j]) * scale
        w = O.rho8(s) / den[j:]
        ds = 8.0 * scale * w / np.sqrt(1.0 + s * s) * (g[j:] @ v[j] - E[j:])
        dk.append(ds @ q[j:])
        dv.append(w @ g[j:])
    return np.array(dq), np.array(dk), np.array(dv)
