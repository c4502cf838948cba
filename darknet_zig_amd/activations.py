"""The activation codes of src/activations.zig:11-56.

The integer values are part of the ABI (they are passed to
dkz_activate_array / dkz_gradient_array) and must keep darknet's order.
"""

from __future__ import annotations

import enum


class Activation(enum.IntEnum):
    logistic = 0
    relu = 1
    relie = 2
    linear = 3
    ramp = 4
    tanh = 5
    plse = 6
    leaky = 7
    elu = 8
    loggy = 9
    stair = 10
    hardtan = 11
    lhtan = 12
    selu = 13

    @classmethod
    def fromString(cls, s: str) -> "Activation":
        """activations.zig:29-51: unknown names fall back to relu."""
        try:
            return cls[s]
        except KeyError:
            return cls.relu

    def toString(self) -> str:
        return self.name
