from .ops import *  # noqa: F401,F403
from .helper import *  # noqa: F401,F403
from .base import *  # noqa: F401,F403
