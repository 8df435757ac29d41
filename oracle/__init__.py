"""CPU oracle for the procedural-IR execution path -- TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker or the
timed CPU baseline.  The product (``ad_amd.device.hip``) never calls it.

``OracleDevice`` restates the reference OpenCL backend
(autodiff/device/opencl/device.py:16-146 and kernels/*.py): the same command
walk, one generated kernel per command with the same statement text, and
the same work decomposition -- one iteration per OpenCL work-item,
sequential fp32 k-loops, the work-group tree reduction with
``L = ceil(R/2)*2`` (including its behaviour for non-power-of-two ``L``).
Kernels are C++ compiled by g++ with OpenMP (one OpenMP iteration per
work-item), ``-ffp-contract=off`` so each statement rounds like a single
OpenCL statement.  Within a fused command every statement completes for
all elements before the next one starts (lockstep), which is the result the
OpenCL kernels give whenever they do not race.

The reference cannot run here (its imports need the absent ``colored`` and
``toposort`` packages, and it needs an OpenCL device), and it contains no
C/C++ to compile, so there is no build of it under ``oracle/_ref``.  What
pins each part of this restatement (tests/test_oracle.py, test_frontend.py):

* dotprod / DPElwFuse: the reference's known answers of
  tests/dotprod_test.py:8-9 (its seeded inputs are fixtures in
  tests/golden/); float64 ``A @ B``.
* unary ops and double literals: tests/unary_test.py:11-14 known answers.
* reduce / ReduceElwFuse / LayerNorm: tests/layernorm_test.py:19-22 known
  answers; float64 LayerNorm forward and gamma/beta gradients; the tree's
  element drops for R = 5, 6 (reduce.py:38-43, TODO.md:43-44).
* contigious / concat / index / pow2: exact values of
  tests/concat_test.py:28-34, powtwo_test.py:18-27, variance_test.py:19-28.
* config-1 MLP training and softmax attention: float64 closed forms.

* ``exact_reduce=True`` (not the reference; the fix of its tree for
  non-power-of-two lengths and of MAX's zero padding): float64 sums and
  exact maxima (test_oracle.py::test_exact_reduce_mode_sums_every_element).

Parity unpinned: ulp-level agreement of ``exp2``/``log2``/``sin`` with the
reference device's libm (its tests round to 4-5 decimals), and the Feeder
offset -- the OpenCL backend writes a Feeder at offset 0
(cl_helper.py:316,326) while the CUDA backend and this oracle use the arena
offset (cuda_helper.py:117-119); ``feeder_offset_zero=True`` reproduces the
OpenCL behaviour.
"""
from .cpu_device import OracleDevice, compile_cpp  # noqa: F401
