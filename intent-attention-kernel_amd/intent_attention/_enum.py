"""String enum whose ``auto()`` value is the member name.

Same value convention as the reference's ``StrEnum`` (_enum.py:5-13): the
metadata the router emits carries upper-case member names (``"FP16"``,
``"INT4_RESIDUAL"``), and ``str(member)`` is that value.
"""
from enum import Enum


class StrEnum(Enum):
    # members are singletons compared by identity: the C-level identity hash
    # agrees with that equality and costs less than Enum's hash of the name
    # (the precision tables look members up on every call)
    __hash__ = object.__hash__

    @staticmethod
    def _generate_next_value_(name, start, count, last_values):  # noqa: D401
        return name

    def __str__(self) -> str:
        return self.value

    def __repr__(self) -> str:
        return f"{type(self).__name__}.{self.value}"
