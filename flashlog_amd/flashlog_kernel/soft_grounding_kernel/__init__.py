"""Graph-guided rule sampling and training-source preparation on gfx950
(the export list of flashlog_kernel/soft_grounding_kernel/__init__.py:1-10)."""
from .soft_grounding_kernel import (
    ground_head_batch_source_folds_sampled_capped_counts,
    sample_relation_sources_reservoir,
)

__all__ = [
    "ground_head_batch_source_folds_sampled_capped_counts",
    "sample_relation_sources_reservoir",
]
