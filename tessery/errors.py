"""tessery's stable error classes (src/metal_inference/errors.py, src/tessery/errors.py)."""

from tessery_amd.errors import *  # noqa: F401,F403
from tessery_amd.errors import __all__  # noqa: F401
