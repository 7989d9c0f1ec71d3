from .schema import detect_graph_mode, load_config, validate_config

__all__ = ["detect_graph_mode", "load_config", "validate_config"]
