"""MI355X-native Avey and Avey-B forward contextualizer (drop-in for avey_kernels)."""

from .ops import avey, avey_b

__all__ = ['avey', 'avey_b']
