"""MI355X-native CPAB transformations (drop-in for FG-CPAB's ``cpab`` package)."""
from .cpab import Cpab

__all__ = ['Cpab']
