"""SO(2) irreps as complex numbers and the flat field layout (the reference's
``gm_attention.representations``)."""

from gm_attention_amd.representations import so2
from gm_attention_amd.representations.field_type import SO2FeatureField, SO2FieldType

__all__ = ["SO2FeatureField", "SO2FieldType", "so2"]
