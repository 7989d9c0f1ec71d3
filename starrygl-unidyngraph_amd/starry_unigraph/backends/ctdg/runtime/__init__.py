from .data import CTDGDataBatch, TGTemporalDataset
from .factory import build_ctdg_runtime
from .memory import CTDGMemoryBank
from .models import CTDGLinkPredictor, CTDGMemoryUpdater, TemporalTransformerConv, build_ctdg_model
from .runtime import CTDGOnlineRuntime
from .sampler import CTDGSampleOutput, NativeTemporalSampler
from .session import CTDGSession

__all__ = ["CTDGDataBatch", "TGTemporalDataset", "build_ctdg_runtime", "CTDGMemoryBank", "CTDGLinkPredictor",
           "CTDGMemoryUpdater", "TemporalTransformerConv", "build_ctdg_model", "CTDGOnlineRuntime",
           "CTDGSampleOutput", "NativeTemporalSampler", "CTDGSession"]
