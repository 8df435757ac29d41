"""Graph IR node kinds (autodiff/graph/)."""
from .compute import *  # noqa: F401,F403
from .control import *  # noqa: F401,F403
from .data import *  # noqa: F401,F403
from .tensor import *  # noqa: F401,F403
from ..node import Node  # noqa: F401
