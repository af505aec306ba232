"""Op bindings (reference: torchpairwise/ops/__init__.py)."""
from .cpdist import *  # noqa: F401,F403
from .metrics import *  # noqa: F401,F403
