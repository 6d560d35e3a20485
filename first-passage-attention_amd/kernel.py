"""Drop-in module name of the reference (``from kernel import ...``): re-exports the fpa API."""
from fpa import Field, FirstPassageAttention, first_passage_attention, first_passage_bias  # noqa: F401
