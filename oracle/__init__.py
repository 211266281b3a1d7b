"""CPU oracle of the ops: a NumPy float64 restatement of the reference's `ref64` / `ref_select64` / `allowed`,
and of the same attention for this build's decode, paged-decode and paged-prefix ops.

TEST INFRASTRUCTURE ONLY.  Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may
import this package, and only as the checker (or, for the CPU baseline, as the thing timed on the host).  The product
path (`vmk`, the kernel modules, libvmk.so) never imports or calls it.

Every function cites the reference file:line it restates.  The restatement uses float64 matrix products (BLAS)
instead of the reference's `np.einsum`; the arithmetic is the same up to float64 summation order.

Pinning (tests/test_oracle.py): float64 SDPA of PyTorch on the CPU as an independent library routine, closed forms
(q = 0 gives the mean of V over the allowed keys, constant V rows, a single allowed key), the cascade/LSE identity,
brute-force sorting for the top-k, and planted mistakes that each of those checks must catch.
"""
from . import prefix, prefix_paged, spec, dsa, decode, decode_paged, dsa_project  # noqa: F401
