"""Write the golden vectors in tests/golden/*.npz.

The reference (tile-rs) is Rust-only, has no executable numeric path for these
ops and no numeric golden vectors of its own (all its tests are text
comparisons), and no Rust toolchain exists here.  These vectors therefore come
from an independent implementation of the same mathematics — PyTorch's CPU
kernels, run in float64 — on small seeded inputs, and they pin the C oracle:

  softmax_f32.npz      linalg.softmax dimension(1)        (mlir_to_linalg.rs:1305-1343)
  matmul_bf16.npz      linalg.fill 0 + linalg.matmul      (mlir_to_linalg.rs:1345-1393)
  matmul_f16_t.npz     same with B stored N x K           (tile.rs:2028)
  attention_f32.npz    transpose/matmul/scale/softmax/matmul (mlir_to_linalg.rs:1781-1902)
  prefill_bf16.npz     causal GQA prefill                  (mlir_to_msl.rs:10928-11009)
  decode_bf16.npz      GQA decode                          (mlir_to_msl.rs:10747-10816)
  rms_norm_f32.npz     RMSNorm, torch.nn.functional.rms_norm (mlir_to_linalg.rs:1666-1763)
  swiglu_bf16.npz      silu(A.B) * UP, torch.nn.functional.silu (mlir_to_linalg.rs:774-782, :425)

Inputs are stored exactly as the kernels see them (f32, or bf16/f16 bit
patterns as uint16); expected outputs are float64 results rounded to f32.
Run: python tests/golden/make_golden.py [case ...]   (CPU only; torch is not needed
anywhere else; with no arguments every case is written)
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16).copy()


def f16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.float16).view(torch.int16).numpy().view(np.uint16).copy()


def softmax_case():
    g = torch.Generator().manual_seed(11)
    x = torch.randn(4, 1024, generator=g, dtype=torch.float32) * 2.0
    x[1] = 3.5  # constant row -> 1/C
    y = torch.softmax(x.double(), dim=1).float()
    np.savez(HERE / "softmax_f32.npz", x=x.numpy(), y=y.numpy())


def matmul_case():
    g = torch.Generator().manual_seed(12)
    m, k, n = 64, 96, 80
    a = (torch.rand(m, k, generator=g) * 2 - 1).to(torch.bfloat16)
    b = (torch.rand(k, n, generator=g) * 2 - 1).to(torch.bfloat16)
    c = (a.double() @ b.double()).float()
    np.savez(HERE / "matmul_bf16.npz", a=bf16_bits(a), b=bf16_bits(b), c=c.numpy(),
             mkn=np.array([m, k, n]))
    a = torch.randn(m, k, generator=g).to(torch.float16)
    bt = (torch.randn(n, k, generator=g) * 0.02).to(torch.float16)
    c = (a.double() @ bt.double().T).float()
    np.savez(HERE / "matmul_f16_t.npz", a=f16_bits(a), b=f16_bits(bt), c=c.numpy(),
             mkn=np.array([m, k, n]))


def attention_case():
    g = torch.Generator().manual_seed(13)
    s, d = 128, 64
    q, k, v = (torch.randn(s, d, generator=g) for _ in range(3))
    o = torch.nn.functional.scaled_dot_product_attention(q.double()[None], k.double()[None],
                                                         v.double()[None])[0].float()
    np.savez(HERE / "attention_f32.npz", q=q.numpy(), k=k.numpy(), v=v.numpy(), o=o.numpy(),
             sd=np.array([s, d]))


def prefill_case():
    g = torch.Generator().manual_seed(14)
    B, S, NH, NKV, D = 2, 96, 4, 2, 128
    start, max_seq = 16, 128  # chunked prefill: 16 cached positions before this chunk
    q = torch.randn(B, S, NH, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, NKV, max_seq, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, NKV, max_seq, D, generator=g).to(torch.bfloat16)
    kv_len = start + S
    qd = q.double().permute(0, 2, 1, 3)                        # B NH S D
    kd = k.double()[:, :, :kv_len].repeat_interleave(NH // NKV, dim=1)
    vd = v.double()[:, :, :kv_len].repeat_interleave(NH // NKV, dim=1)
    # query i sits at absolute position start + i and sees positions <= start + i
    mask = torch.arange(kv_len)[None, :] <= (start + torch.arange(S))[:, None]
    o = torch.nn.functional.scaled_dot_product_attention(qd, kd, vd, attn_mask=mask)
    o = o.permute(0, 2, 1, 3).float()                           # B S NH D
    np.savez(HERE / "prefill_bf16.npz", q=bf16_bits(q), k=bf16_bits(k), v=bf16_bits(v),
             o=o.numpy(), shape=np.array([B, S, start, max_seq, D, NH, NKV]))


def decode_case():
    g = torch.Generator().manual_seed(15)
    B, NH, NKV, D, L, max_seq = 2, 8, 2, 128, 300, 320
    q = torch.randn(B, NH, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, NKV, max_seq, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, NKV, max_seq, D, generator=g).to(torch.bfloat16)
    qd = q.double()[:, :, None, :]
    kd = k.double()[:, :, :L].repeat_interleave(NH // NKV, dim=1)
    vd = v.double()[:, :, :L].repeat_interleave(NH // NKV, dim=1)
    o = torch.nn.functional.scaled_dot_product_attention(qd, kd, vd)[:, :, 0, :].float()
    np.savez(HERE / "decode_bf16.npz", q=bf16_bits(q), k=bf16_bits(k), v=bf16_bits(v),
             o=o.numpy(), shape=np.array([B, L, max_seq, D, NH, NKV]))


def rms_norm_case():
    g = torch.Generator().manual_seed(16)
    x = torch.randn(6, 768, generator=g, dtype=torch.float32) * 3.0
    x[2] = -0.75                 # constant row -> -0.75 / sqrt(0.5625 + eps)
    x[4] = 0.0
    x[4, 17] = 5.0               # one-hot row
    eps = 1e-5
    y = torch.nn.functional.rms_norm(x.double(), (768,), eps=eps).float()
    np.savez(HERE / "rms_norm_f32.npz", x=x.numpy(), y=y.numpy(), eps=np.array([eps]))


def swiglu_case():
    g = torch.Generator().manual_seed(17)
    m, k, n = 48, 64, 72
    a = torch.randn(m, k, generator=g).to(torch.bfloat16)
    b = (torch.randn(k, n, generator=g) * 0.3).to(torch.bfloat16)
    up = torch.randn(m, n, generator=g, dtype=torch.float32)
    c = (torch.nn.functional.silu(a.double() @ b.double()) * up.double()).float()
    np.savez(HERE / "swiglu_bf16.npz", a=bf16_bits(a), b=bf16_bits(b), up=up.numpy(), c=c.numpy(),
             mkn=np.array([m, k, n]))


CASES = {"softmax": softmax_case, "matmul": matmul_case, "attention": attention_case,
         "prefill": prefill_case, "decode": decode_case, "rms_norm": rms_norm_case,
         "swiglu": swiglu_case}

if __name__ == "__main__":
    import sys
    for name in (sys.argv[1:] or list(CASES)):
        CASES[name]()
    for p in sorted(HERE.glob("*.npz")):
        print(p.name, p.stat().st_size)
