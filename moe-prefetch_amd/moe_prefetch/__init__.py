"""MI355X-native MoE decode hot path (router + slot cache + Q4_K/Q6_K experts).

Drop-in surfaces of the reference's Python prototypes:
  ExpertCache      (src/prefetch_engine.py)
  ExpertPredictor  (src/predictor.py)
The engine itself (the llama-moecache runtime and the expert kernels) is
MoeCache; all of it calls libmoeprefetch.so through its C ABI.
"""
from ._lib import MoeError, TYPE_Q4K, TYPE_Q6K, lib
from .engine import MoeCache, parse_slot_profile
from .predictor import ExpertPredictor
from .prefetch_engine import ExpertCache

__all__ = ["ExpertCache", "ExpertPredictor", "MoeCache", "MoeError", "TYPE_Q4K", "TYPE_Q6K",
           "lib", "parse_slot_profile"]
