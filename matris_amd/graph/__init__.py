from .converter import GraphConverter
from .radiusgraph import RadiusGraph, datatype

__all__ = ["GraphConverter", "RadiusGraph", "datatype"]
