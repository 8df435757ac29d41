"""MI355X backend for the procedural IR (mirrors autodiff/device/opencl/)."""
from .device import HIPDevice  # noqa: F401
