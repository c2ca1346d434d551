"""Device-side seeded synthetic GGUF weights for large GPU tests and the bench
(torch's counter-based generator on the GPU: the bytes are deterministic for a
seed on a given device, and tests hand the same bytes to the oracle)."""
from __future__ import annotations

Q4_K, IQ4_XS = 3, 15  # SchemeId codes (r9v_amd.ffi)
BLOCK_BYTES = {Q4_K: 144, IQ4_XS: 136}


def quant_weights_gpu(torch, scheme, seed, rows, k, device="cuda"):
    """uint8 [rows, k/256*block_bytes] GGUF blocks: uniform payload/scale
    bytes, d (and dmin) = f16(|N(0, 0.02)|) (|N(0, 0.01)|)."""
    bb = BLOCK_BYTES[scheme]
    nblocks = rows * (k // 256)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    blk = torch.randint(0, 256, (nblocks, bb), dtype=torch.uint8, generator=g, device=device)
    d = (torch.randn(nblocks, generator=g, device=device) * 0.02).abs().half()
    blk[:, 0:2] = d.view(torch.uint8).view(nblocks, 2)
    if scheme == Q4_K:
        dmin = (torch.randn(nblocks, generator=g, device=device) * 0.01).abs().half()
        blk[:, 2:4] = dmin.view(torch.uint8).view(nblocks, 2)
    return blk.view(rows, (k // 256) * bb)
