from .neighbors import *  # noqa: F401,F403
from .pairwise import *  # noqa: F401,F403
