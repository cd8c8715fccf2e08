"""Always-active shared expert (mirrors ResidentSharedExpert, src/vesper/shared.py:141-170).

The decode layer stores the shared expert in MXFP4 next to the routed experts
and runs it through the same kernels, unweighted, added last by the combine.
"""

from __future__ import annotations

from .expert import ResidentExpert


class ResidentSharedExpert(ResidentExpert):
    """forward(x) = expert(x) with no routing weight (shared.py:169-170)."""

    def forward(self, x, routing_weight=None) -> dict:
        if routing_weight is not None:
            raise ValueError("The shared expert is never routing-weighted")
        return self.execute(x, self.weights, None)
