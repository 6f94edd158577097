from .scheduler import Scheduler, SequenceStatus, StreamResult

__all__ = ["Scheduler", "SequenceStatus", "StreamResult"]
