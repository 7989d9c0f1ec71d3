from .time_encode import TimeEncode

__all__ = ["TimeEncode"]
