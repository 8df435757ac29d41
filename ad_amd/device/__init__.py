class Device:
    """Backend base class (autodiff/device/__init__.py:1-6)."""

    def __init__(self):
        return None

    def execute(self, proc):
        raise NotImplementedError("Device not execute error")
