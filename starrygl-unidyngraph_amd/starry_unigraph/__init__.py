"""starry_unigraph -- MI355X-native CTDG training step (temporal sampler,
memory/mailbox update, time encoding + temporal attention) behind the
reference's API (SchedulerSession, ctdg.pipeline: online, the native sampler
binding)."""
__version__ = "0.1.1+mi355x"


def __getattr__(name):
    if name == "SchedulerSession":
        from .session import SchedulerSession
        return SchedulerSession
    raise AttributeError(name)
