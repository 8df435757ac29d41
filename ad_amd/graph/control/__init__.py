from .ir_for import *  # noqa: F401,F403
