"""Drop-in module name of the reference's src/prefetch_engine.py."""
from moe_prefetch.prefetch_engine import EXPERT_BYTES, EXPERT_MIB, ExpertCache  # noqa: F401
