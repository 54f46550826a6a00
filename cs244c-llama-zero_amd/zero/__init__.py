from .stage0_ddp import ZeROStage0DDP
from .stage1_optimizer import ZeROStage1Optimizer
from .stage2_optimizer import ZeROStage2Optimizer
from .stage3_optimizer import ZeROStage3Optimizer

__all__ = [
    "ZeROStage0DDP",
    "ZeROStage1Optimizer",
    "ZeROStage2Optimizer",
    "ZeROStage3Optimizer",
]
