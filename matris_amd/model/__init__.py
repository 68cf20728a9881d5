from .model import MatRIS

__all__ = ["MatRIS"]
