"""MI355X (gfx950) implementation of CompactLogic's logic-layer hot path.

Same public modules as the reference package `compactlogic` (compactlogic/__init__.py:1):
LogicLayer, GroupSum and the autograd bridge LogicLayerCudaFunction, plus the packed-bit
inference API (PackBitsTensor).  All numerics run in libcompactlogic_hip.so, built in-tree by
``python -m compactlogic_amd.build``.
"""
from . import difflogic_hip
from .layers import (GroupSum, GroupSumFunction, LogicLayer, LogicLayerCudaFunction,
                     LogicLayerRunsFunction, PackBitsTensor)
from .plan import RunPlan, build_run_plan

__all__ = [
    "LogicLayer", "GroupSum", "LogicLayerCudaFunction", "LogicLayerRunsFunction",
    "GroupSumFunction", "PackBitsTensor", "RunPlan", "build_run_plan", "difflogic_hip",
]
