"""Objective configuration, field-identical to the reference's ``Objective``.

Reference: nanospec/config.py:54-66.  ``asdict(objective)`` is part of the
reference's checkpoint identity (checkpoint.py:39, 68-69), so the fields, their
order, defaults and validation errors are kept exactly; kernel options live in
keyword arguments of the entry points instead.
"""

from dataclasses import dataclass


@dataclass
class Objective:
    block_size: int = 7
    num_anchors: int = 32
    gamma: float = 4.0
    ce: float = 0.1
    kl: float = 0.9

    def __post_init__(self):
        if self.block_size < 1 or self.num_anchors < 1:
            raise ValueError("block_size and num_anchors must be positive")
        if min(self.ce, self.kl) < 0:
            raise ValueError("Loss weights must be nonnegative")
