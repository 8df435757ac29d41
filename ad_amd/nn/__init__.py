from .activations import *  # noqa: F401,F403
from .linear import *  # noqa: F401,F403
from .sequential import *  # noqa: F401,F403
from .module import *  # noqa: F401,F403
from .transformer import *  # noqa: F401,F403
from .optimizers import *  # noqa: F401,F403
from .normalization import *  # noqa: F401,F403
