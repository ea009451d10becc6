"""Helpers shared by the GPU parity tests."""
import numpy as np


def tdev(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def from_bits16(bits, kind):
    """uint16 bit array -> torch f16/bf16 tensor on the GPU."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda()
    return t.view(torch.float16 if kind == "f16" else torch.bfloat16)


def host(t):
    import torch
    if t.dtype == torch.bfloat16:
        return t.float().cpu().numpy().astype(np.float64)
    return t.cpu().numpy().astype(np.float64)


def rel_err(got, ref, floor=1e-2):
    """Elementwise error relative to |ref| plus a floor of ``floor`` x rms(ref)
    (keeps near-zero outputs from dominating); returns the max."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denom = np.abs(ref) + floor * np.sqrt(np.mean(ref ** 2) + 1e-300)
    return float(np.max(np.abs(got - ref) / denom))


def assert_close(got, ref, rtol=1e-3, what=""):
    e = rel_err(got, ref)
    assert e <= rtol, f"{what}: max relative error {e:.3e} > {rtol:.1e}"
    return e


def assert_close_f16(got, ref_f64, rtol=1e-3, what=""):
    """An f16-stored output against the float64 oracle: each element within
    the assert_close bar of the f16-rounded oracle value, or one f16 ulp of
    it (the kernel's float32 sum and the float64 one may straddle a rounding
    edge; near zero one ulp can exceed the relative bar)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref_f64, dtype=np.float64)
    r16 = ref.astype(np.float16).astype(np.float64)
    denom = np.abs(r16) + 1e-2 * np.sqrt(np.mean(r16 ** 2) + 1e-300)
    e = np.abs(got - r16)
    mag = np.maximum(np.abs(ref), 2.0 ** -14)
    ulp = 2.0 ** (np.floor(np.log2(mag)) - 10)
    bad = (e > rtol * denom) & (e > ulp * (1 + 1e-9))
    assert not bad.any(), (f"{what}: {bad.sum()} elements beyond the bar and one f16 ulp "
                           f"(max rel {float(np.max(e / denom)):.3e})")


def assert_close_normwise(got, ref, rtol=1e-3, what=""):
    """End-to-end bar for decoder logits: max|got - ref| <= rtol * max|ref|.

    After several layers of f16 storage rounding, fp32-vs-fp64 differences
    flip individual f16 roundings and the flips propagate; an fp32 CPU
    evaluation of the same algorithm deviates from the fp64 oracle by
    ~3.6e-4 of max|logit| on the tiny model, so the per-element bar of
    assert_close does not apply end to end.  Greedy tokens must still be
    identical."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    e = float(np.max(np.abs(got - ref)) / np.max(np.abs(ref)))
    assert e <= rtol, f"{what}: max |err| / max |ref| = {e:.3e} > {rtol:.1e}"
    return e


def assert_bf16_faithful(got, ref_f64, what="", sum_err=0.0):
    """Reference Q4 outputs are BF16-truncated fp32 sums.  The GPU's fp32 sum
    and the fp64 oracle may straddle a truncation boundary, so the bar is one
    bf16 ulp (2^-7 relative) plus exact bf16-representability of the output.
    ``sum_err``: a bound on the fp32 summation error itself (scalar or per
    element), which matters where the sum cancels to near zero."""
    from oracle import oracle as O
    got = np.asarray(got, dtype=np.float64)
    normal = np.abs(got) >= 2.0 ** -14          # f16 subnormals round once more
    assert np.array_equal(O.bf16_trunc(got[normal]), got[normal]), \
        f"{what}: output not bf16-truncated"
    ref_t = O.bf16_trunc(ref_f64)
    bound = 2.0 ** -7 * np.abs(ref_f64) + 2.0 ** -24 + sum_err
    bad = np.abs(got - ref_t) > bound
    assert not bad.any(), f"{what}: {bad.sum()} elements differ by more than one bf16 ulp"
