from .checks import check_D

__all__ = ["check_D"]
