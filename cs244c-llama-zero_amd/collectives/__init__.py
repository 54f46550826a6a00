from .interface import CollectiveOps, LocalCollectives, SendRecvCollectives, TorchCollectives, TracingCollectives

__all__ = [
    "CollectiveOps",
    "LocalCollectives",
    "SendRecvCollectives",
    "TorchCollectives",
    "TracingCollectives",
]
