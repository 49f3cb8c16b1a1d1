from .isoquant import IsoQuantMSE, make_random_unit_quaternion
from .lloyd_max import LloydMaxCodebook, solve_lloyd_max
from .planarquant import PlanarQuantMSE, make_random_rotations

__all__ = ["LloydMaxCodebook", "IsoQuantMSE", "PlanarQuantMSE", "solve_lloyd_max",
           "make_random_unit_quaternion", "make_random_rotations"]
