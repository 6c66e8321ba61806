"""Seeded synthetic workloads for the benchmark configurations.

IQ3_S blocks: d = fp16(|N(0,1)| * 0.02); every other byte uniform, which
makes grid indices uniform over 0..511, sign bits uniform and the 4-bit
sub-block scales uniform over 0..15.  Q8_0 blocks: d = fp16(|N(0,1)| * 0.01),
int8 values uniform over -127..127.  Activations and router logits are fp32
N(0,1); the prefill router adds a Zipf(s=1.1) popularity bias
-1.1 * ln(rank(e)) with rank a seeded permutation of 1..E.

Host generators (numpy) define the data the parity tests use; the device
generators (torch) build the same distributions in HBM for the benchmark's
multi-GB layer stacks.
"""
import numpy as np

T_Q8_0 = 8
T_IQ3_S = 21


def iq3s_bytes(rng, nblocks):
    b = rng.integers(0, 256, size=(nblocks, 110), dtype=np.uint8)
    d = (np.abs(rng.standard_normal(nblocks)) * 0.02).astype(np.float16)
    b[:, 0:2] = d.view(np.uint8).reshape(nblocks, 2)
    return b.reshape(-1)


def q80_bytes(rng, nblocks):
    b = np.empty((nblocks, 34), np.uint8)
    d = (np.abs(rng.standard_normal(nblocks)) * 0.01).astype(np.float16)
    b[:, 0:2] = d.view(np.uint8).reshape(nblocks, 2)
    b[:, 2:] = rng.integers(-127, 128, size=(nblocks, 32), dtype=np.int8).view(np.uint8)
    return b.reshape(-1)


T_Q6_K, T_IQ4_NL, T_IQ2_S, T_Q2_0 = 14, 20, 22, 42
T_IQ2_XXS, T_IQ2_XS, T_IQ3_XXS, T_IQ4_XS = 16, 17, 18, 23
# (values per block, bytes per block, offset of the fp16 scale)
BLOCKS = {T_IQ3_S: (256, 110, 0), T_Q8_0: (32, 34, 0), T_IQ4_NL: (32, 18, 0),
          T_Q2_0: (64, 18, 0), T_IQ2_S: (256, 82, 0), T_Q6_K: (256, 210, 208),
          T_IQ2_XXS: (256, 66, 0), T_IQ2_XS: (256, 74, 0), T_IQ3_XXS: (256, 98, 0),
          T_IQ4_XS: (256, 136, 0)}


def blocks_bytes(rng, ty, nblocks):
    """Uniform bytes with an fp16 |N(0,1)| * 0.02 block scale: every field of
    these formats (indices, signs, sub-block scales, quants) is then uniform
    over its range."""
    vals, nb, doff = BLOCKS[ty]
    b = rng.integers(0, 256, size=(nblocks, nb), dtype=np.uint8)
    d = (np.abs(rng.standard_normal(nblocks)) * 0.02).astype(np.float16)
    b[:, doff:doff + 2] = d.view(np.uint8).reshape(nblocks, 2)
    return b.reshape(-1)


def matrix(rng, ty, rows, cols):
    if ty == T_IQ3_S:
        return iq3s_bytes(rng, rows * cols // 256)
    if ty == T_Q8_0:
        return q80_bytes(rng, rows * cols // 32)
    return blocks_bytes(rng, ty, rows * cols // BLOCKS[ty][0])


def expert_stride(n_embd, n_ff, ty=T_IQ3_S):
    """Packed expert = gate[n_ff][n_embd] | up | down[n_embd][n_ff]."""
    if ty == T_IQ3_S:
        rg, rd = n_embd // 256 * 110, n_ff // 256 * 110
    else:
        rg, rd = n_embd // 32 * 34, n_ff // 32 * 34
    return 2 * n_ff * rg + n_embd * rd, 0, n_ff * rg, 2 * n_ff * rg


def expert_arena(rng, n_exp, n_embd, n_ff, ty=T_IQ3_S):
    """n_exp packed experts back to back (IQ3_S: every part is whole
    110-byte blocks, so the arena is one block sequence)."""
    stride = expert_stride(n_embd, n_ff, ty)[0]
    if ty == T_IQ3_S:
        return iq3s_bytes(rng, n_exp * stride // 110)
    return q80_bytes(rng, n_exp * stride // 34)


def zipf_bias(rng, n_exp, s=1.1):
    rank = rng.permutation(n_exp) + 1
    return (-s * np.log(rank)).astype(np.float32)


def logits(rng, T, n_exp, zipf=False):
    lg = rng.standard_normal((T, n_exp)).astype(np.float32)
    if zipf:
        lg = lg + zipf_bias(rng, n_exp)[None, :]
    return lg


# ---------------------------------------------------------------- device side

def device_iq3s(nbytes, seed, device="cuda"):
    """IQ3_S block bytes (nbytes multiple of 110) generated in HBM."""
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    nb = nbytes // 110
    b = torch.randint(0, 256, (nb, 110), dtype=torch.uint8, device=device, generator=g)
    d = (torch.randn(nb, device=device, generator=g).abs() * 0.02).to(torch.float16)
    b[:, 0:2] = d.view(torch.uint8).view(nb, 2)
    return b.view(-1)


def device_blocks(ty, nblocks, seed, device="cuda"):
    """Blocks of any format in BLOCKS generated in HBM: uniform bytes with an
    fp16 |N(0,1)| * 0.02 block scale (every index, sign, sub-block scale and
    quant field then uniform over its range)."""
    import torch
    vals, nb, doff = BLOCKS[ty]
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    b = torch.randint(0, 256, (nblocks, nb), dtype=torch.uint8, device=device, generator=g)
    d = (torch.randn(nblocks, device=device, generator=g).abs() * 0.02).to(torch.float16)
    b[:, doff:doff + 2] = d.view(torch.uint8).view(nblocks, 2)
    return b.view(-1)


def device_q80(nbytes, seed, device="cuda"):
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    nb = nbytes // 34
    b = torch.empty((nb, 34), dtype=torch.uint8, device=device)
    d = (torch.randn(nb, device=device, generator=g).abs() * 0.01).to(torch.float16)
    b[:, 0:2] = d.view(torch.uint8).view(nb, 2)
    b[:, 2:] = torch.randint(-127, 128, (nb, 32), dtype=torch.int8, device=device,
                             generator=g).view(torch.uint8)
    return b.view(-1)
