"""MI355X (gfx950) implementation of CompactLogic's logic-layer hot path.

Same public modules as the reference package `compactlogic` (compactlogic/__init__.py:1):
LogicLayer, ConvLayer, GroupSum and the autograd bridges LogicLayerCudaFunction and
ConvLayerCudaFunction, plus the packed-bit inference API (PackBitsTensor), and the logic-tree
conv blocks of the third-party ConvLogic package (ConvLogicLayer, TreeLogicLayer,
PoolLogicLayer).  All numerics run in libcompactlogic_hip.so, built in-tree by
``python -m compactlogic_amd.build``.
"""
from . import checkpoint, circuit, convlogic_hip, difflogic_hip
from .layers import (ConvLayer, ConvLayerCudaFunction, ConvLayerSoftmaxFunction,
                     ConvLayerWindowFunction, GroupSum, GroupSumCrossEntropyFunction,
                     GroupSumFunction, LogicGroupSumCrossEntropyFunction, LogicLayer,
                     LogicLayerCudaFunction, LogicLayerRunsFunction, PackBitsTensor,
                     logic_group_sum_cross_entropy, sequential_cross_entropy)
from .optim import FusedAdam
from .packed_net import PackedNetwork
from .plan import RunPlan, build_run_plan
from .schedules import (EntropyRowResampler, FixedSequentialEntropyFreezer,
                        SequentialEntropyFreezer)
from .treelogic import (ConvLogicFunction, ConvLogicLayer, FullConvLogicFunction,
                        PoolLogicLayer, TreeLogicFunction, TreeLogicLayer)

__all__ = [
    "LogicLayer", "GroupSum", "LogicLayerCudaFunction", "LogicLayerRunsFunction",
    "GroupSumCrossEntropyFunction", "GroupSumFunction", "PackBitsTensor", "RunPlan", "build_run_plan", "difflogic_hip",
    "ConvLayer", "ConvLayerCudaFunction", "ConvLayerSoftmaxFunction", "ConvLayerWindowFunction",
    "convlogic_hip", "SequentialEntropyFreezer", "FixedSequentialEntropyFreezer",
    "EntropyRowResampler", "PackedNetwork", "ConvLogicLayer", "TreeLogicLayer", "PoolLogicLayer",
    "ConvLogicFunction", "FullConvLogicFunction", "TreeLogicFunction", "FusedAdam",
    "LogicGroupSumCrossEntropyFunction", "logic_group_sum_cross_entropy",
    "sequential_cross_entropy", "checkpoint", "circuit",
]
