from .mem_opt import *  # noqa: F401,F403
from .dep_opt import *  # noqa: F401,F403
from .repeat_opt import *  # noqa: F401,F403
from .in_place import *  # noqa: F401,F403
