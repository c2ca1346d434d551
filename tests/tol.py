"""The north-star matmul tolerance: |gpu - ref| <= 1e-3 * max|ref| + 2e-3 * |ref| per element."""
import numpy as np

ABS_OF_MAX = 1e-3
REL = 2e-3


def check_close(got, ref, what=""):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    bound = ABS_OF_MAX * np.max(np.abs(ref)) + REL * np.abs(ref)
    err = np.abs(got - ref)
    bad = err > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} elements out of tolerance; "
                           f"worst err {float(err.max()):.3e} vs max|ref| {float(np.abs(ref).max()):.3e}")
    return float((err / np.maximum(np.max(np.abs(ref)), 1e-30)).max())


def check_bf16_out(got_bf16_as_f32, got_f32, ref_f32, what=""):
    """bf16 outputs.  T0 writes bf16(acc) (crates/r9v-t0/src/dtype.rs:102-111)
    and one bf16 ulp (2^-8 relative) is larger than the 2e-3 relative term,
    so the tolerance is applied where it is meaningful: the kernel's f32
    accumulator (the same launch with an f32 output) must be within tolerance
    of the oracle's f32 accumulator, and the bf16 output must be exactly the
    round-to-nearest-even of that accumulator.  The fraction of bf16 outputs
    equal to the oracle's own bf16 is returned (only rounding-boundary
    straddles differ)."""
    from r9v_amd import synth

    check_close(got_f32, ref_f32, what)
    want = synth.bf16_bits_to_f32(synth.to_bf16_bits(np.asarray(got_f32, dtype=np.float32)))
    assert np.array_equal(np.asarray(got_bf16_as_f32, dtype=np.float32).view(np.uint32), want.view(np.uint32)), \
        f"{what}: bf16 output is not the RNE of the f32 accumulator"
    ref16 = synth.bf16_bits_to_f32(synth.to_bf16_bits(ref_f32))
    same = float(np.mean(np.asarray(got_bf16_as_f32, dtype=np.float32) == ref16))
    assert same >= 0.8, f"{what}: only {same:.3f} of bf16 outputs equal the oracle's bf16"
    return same
