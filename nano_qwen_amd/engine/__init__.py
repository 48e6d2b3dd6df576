from .model_runner import ModelRunner
from .sequence import Sequence

__all__ = ["ModelRunner", "Sequence"]
