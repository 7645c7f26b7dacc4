"""MI355X-native Avey and Avey-B forward contextualizer (drop-in for avey_kernels)."""

from .ops import avey, avey_b, avey_b_enriched, avey_enriched

__all__ = ['avey', 'avey_b', 'avey_enriched', 'avey_b_enriched']
