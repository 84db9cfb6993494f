"""fmlh_gemm_ex_noalloc: the allocation-free variant of fmlh_gemm_ex (split-K partials in a fixed
device array instead of the grow-on-demand workspace).

Its results must equal fmlh_gemm_ex's bit for bit (same plan, same kernels; only where the
partials live differs), on two calls in a row with the second smaller (the array keeps the
first call's partials), for products that split K on every kernel family and one that does not.
A product whose partials exceed the array is refused; in a child process whose next library
allocation is made to fail (FMLH_FAULT=alloc:1), the no-alloc products still run.
"""
import os
import subprocess
import sys

import numpy as np
import pytest

import freeml_amd as fh

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module", autouse=True)
def device():
    fh.init(0)


def _gemm(fn, A, B, b_trans, epi=fh.EPI_NONE, R=None):
    M, K = A.shape
    N = B.shape[0] if b_trans else B.shape[1]
    dA, dB = fh.DeviceArray.from_host(A), fh.DeviceArray.from_host(B)
    dC = fh.DeviceArray((M, N))
    dR = fh.DeviceArray.from_host(R) if R is not None else None
    fh.call(fn, dA.ptr, K, dB.ptr, B.shape[1], int(b_trans), dC.ptr, N, M, N, K, epi,
            dR.ptr if dR is not None else None, N)
    return dC.numpy()


# (M, N, K, b_trans, epilogue): MFMA tiles with K split for a grid too small for the device,
# skinny NN (M <= 8, K split in 16-row blocks), the NT kernel's two K halves, and products that
# split nothing.
CASES = [(64, 1536, 384, False, fh.EPI_GELU), (8, 1536, 384, False, fh.EPI_RESID),
         (40, 384, 1536, True, fh.EPI_NONE), (5, 384, 1536, False, fh.EPI_NONE),
         (300, 768, 256, True, fh.EPI_GELU), (128, 384, 1536, True, fh.EPI_RESID),
         (512, 1024, 1024, True, fh.EPI_RESID), (4, 384, 384, True, fh.EPI_NONE)]


@pytest.mark.parametrize("first,second", [(0, 1), (2, 3), (4, 5), (6, 0), (0, 7)])
def test_noalloc_equals_gemm_ex_on_two_calls_in_a_row(first, second):
    r = np.random.default_rng(first * 10 + second)
    sizes = []
    for idx in (first, second):
        M, N, K, bt, epi = CASES[idx]
        A = r.standard_normal((M, K)).astype(np.float32)
        B = r.standard_normal((N, K) if bt else (K, N)).astype(np.float32)
        R = r.standard_normal((M, N)).astype(np.float32) if epi == fh.EPI_RESID else None
        print(f"case {idx}: {M}x{N}x{K} b_trans={bt} epilogue={epi}", flush=True)
        got = _gemm("fmlh_gemm_ex_noalloc", A, B, bt, epi, R)
        ref = _gemm("fmlh_gemm_ex", A, B, bt, epi, R)
        np.testing.assert_array_equal(got, ref)
        sizes.append(M * N)
    assert sizes[1] < sizes[0]  # the second call is the smaller one


def test_noalloc_refuses_partials_beyond_its_array():
    A = np.ones((8, 1024), np.float32)
    B = np.ones((1024, 65536), np.float32)  # skinny NN: 64 K blocks x 8 x 65536 partials > 4 Mi floats
    with pytest.raises(fh.FreeMLHipError, match="fixed scratch"):
        _gemm("fmlh_gemm_ex_noalloc", A, B, False)


def test_noalloc_makes_no_library_allocation():
    """In a child process: operand buffers are made first, then FMLH_FAULT=alloc:1 is armed (the
    library's next device allocation fails).  Three no-alloc products of a shape that splits K
    must succeed, since they allocate nothing; fmlh_gemm_ex of the same shape must then hit the
    hook, as its workspace is not allocated yet; disarmed, it gives the same result."""
    script = r"""
import os, sys
import numpy as np
sys.path.insert(0, {root!r})
import freeml_amd as fh
fh.init(0)
r = np.random.default_rng(7)
A = r.standard_normal((64, 384)).astype(np.float32)
B = r.standard_normal((384, 1536)).astype(np.float32)
dA, dB = fh.DeviceArray.from_host(A), fh.DeviceArray.from_host(B)
dC1, dC2 = fh.DeviceArray((64, 1536)), fh.DeviceArray((64, 1536))
os.environ["FMLH_FAULT"] = "alloc:1"
fh.init(0)  # arms the hook
for _ in range(3):
    fh.call("fmlh_gemm_ex_noalloc", dA.ptr, 384, dB.ptr, 1536, 0, dC1.ptr, 1536, 64, 1536, 384, 0, None, 1536)
fh.synchronize()
try:
    fh.call("fmlh_gemm_ex", dA.ptr, 384, dB.ptr, 1536, 0, dC2.ptr, 1536, 64, 1536, 384, 0, None, 1536)
except fh.FreeMLHipError as e:
    assert "FMLH_FAULT" in str(e), e
    print("gemm_ex allocation refused by the hook", flush=True)
else:
    raise AssertionError("fmlh_gemm_ex did not allocate its workspace")
os.environ.pop("FMLH_FAULT")
fh.init(0)
fh.call("fmlh_gemm_ex", dA.ptr, 384, dB.ptr, 1536, 0, dC2.ptr, 1536, 64, 1536, 384, 0, None, 1536)
assert np.array_equal(dC1.numpy(), dC2.numpy())
print("NOALLOC_OK", flush=True)
""".format(root=ROOT)
    env = dict(os.environ)
    env.pop("FMLH_FAULT", None)
    r = subprocess.run([sys.executable, "-u", "-c", script], env=env, capture_output=True, text=True,
                       timeout=180)
    print(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0 and "NOALLOC_OK" in r.stdout
