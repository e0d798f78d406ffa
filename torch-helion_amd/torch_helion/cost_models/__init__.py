"""MI355X hardware description and the roofline cost model used by the planner."""

from .hw_spec import DEFAULT_HW_SPEC, HardwareSpec
from .roofline import CostBreakdown, CostModelError, kernel_cost

__all__ = ["CostBreakdown", "CostModelError", "DEFAULT_HW_SPEC", "HardwareSpec", "kernel_cost"]
