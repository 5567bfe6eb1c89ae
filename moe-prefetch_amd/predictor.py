"""Drop-in module name of the reference's src/predictor.py."""
from moe_prefetch.predictor import N_EXPERT, ExpertPredictor  # noqa: F401
