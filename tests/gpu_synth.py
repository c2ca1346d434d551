"""Device-side seeded synthetic GGUF weights for large GPU tests and the bench
(torch's counter-based generator on the GPU: the bytes are deterministic for a
seed on a given device, and tests hand the same bytes to the oracle)."""
from __future__ import annotations

from r9v_amd.synth import BLOCK_BYTES, BLOCK_LEN, D_OFFSET

Q4_K, IQ4_XS = 3, 15  # SchemeId codes (r9v_amd.ffi)


def quant_weights_gpu(torch, scheme, seed, rows, k, device="cuda"):
    """uint8 [rows, k/block_len*block_bytes] GGUF wire blocks of any of the
    five schemes: uniform payload/scale bytes, each block's f16 d (at its
    scheme's offset) = f16(|N(0, 0.02)|), Q4_K's dmin f16(|N(0, 0.01)|)."""
    bb, bl = BLOCK_BYTES[scheme], BLOCK_LEN[scheme]
    nblocks = rows * (k // bl)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    blk = torch.randint(0, 256, (nblocks, bb), dtype=torch.uint8, generator=g, device=device)
    d = (torch.randn(nblocks, generator=g, device=device) * 0.02).abs().half()
    o = D_OFFSET[scheme]
    blk[:, o:o + 2] = d.view(torch.uint8).view(nblocks, 2)
    if scheme == Q4_K:
        dmin = (torch.randn(nblocks, generator=g, device=device) * 0.01).abs().half()
        blk[:, 2:4] = dmin.view(torch.uint8).view(nblocks, 2)
    return blk.view(rows, (k // bl) * bb)
