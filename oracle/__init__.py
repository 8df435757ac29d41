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
OpenCL statement.

Deliberate difference: a Feeder writes at its arena offset (the CUDA
backend's behaviour, cuda_helper.py:117-119); the OpenCL backend passes
offset 0 (cl_helper.py:316,326), which lands inputs in the wrong place
whenever the Feeder is not at offset 0.  ``feeder_offset_zero=True``
reproduces the OpenCL behaviour.
"""
from .cpu_device import OracleDevice, compile_cpp  # noqa: F401
