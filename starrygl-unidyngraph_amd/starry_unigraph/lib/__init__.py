from .loader import load_bts_sampler_module

__all__ = ["load_bts_sampler_module"]
