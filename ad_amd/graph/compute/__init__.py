from .binary import *  # noqa: F401,F403
from .dotprod import *  # noqa: F401,F403
from .reduce import *  # noqa: F401,F403
from .unary import *  # noqa: F401,F403
