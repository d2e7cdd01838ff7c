"""CPU oracle of the burn-rocket op surface — test infrastructure (see oracle.py)."""
from .oracle import *  # noqa: F401,F403
from .oracle import lib, LIB_PATH  # noqa: F401
