"""flashlog_amd: FlashLog's sparse rule-propagation hot path for MI355X (gfx950).

``flashlog_amd.flashlog_kernel`` mirrors the reference package
``flashlog_kernel`` (same public names and signatures).  ``install()``
registers it under the reference's module names so unchanged model files
(``from flashlog_kernel.flashlog_kernel import dense_csr_sum_cuda``) use it.
"""
import sys

__version__ = "0.1.0"


def install(rules=False):
    """Alias ``flashlog_kernel``, ``flashlog_kernel.flashlog_kernel`` and
    ``flashlog_kernel.soft_grounding_kernel[.soft_grounding_kernel]`` to this
    package's mirrors (drop-in replacement of the reference package).
    rules=True also redirects ``rules.shared_inference``,
    ``rules.max_inference`` (their ``score`` entry points) and
    ``rules.evaluate`` (the rule-evaluation primitives and scorer) to the GPU
    rule-bank scoring and ``rules.indexed_bank`` to this package's indexed
    rule bank, leaving the rest of a ``rules`` package alone."""
    from . import flashlog_kernel as pkg
    from .flashlog_kernel import flashlog_kernel as mod
    from .flashlog_kernel import soft_grounding_kernel as sg
    from .flashlog_kernel.soft_grounding_kernel import soft_grounding_kernel as sgm
    sys.modules["flashlog_kernel"] = pkg
    sys.modules["flashlog_kernel.flashlog_kernel"] = mod
    sys.modules["flashlog_kernel.soft_grounding_kernel"] = sg
    sys.modules["flashlog_kernel.soft_grounding_kernel.soft_grounding_kernel"] = sgm
    if rules:
        from .rules import evaluate as evm, indexed_bank as ib, max_inference as mi, shared_inference as si
        sys.modules["rules.indexed_bank"] = ib
        sys.modules["rules.shared_inference"] = si
        sys.modules["rules.max_inference"] = mi
        sys.modules["rules.evaluate"] = evm
        parent = sys.modules.get("rules")
        if parent is not None:
            parent.shared_inference, parent.max_inference, parent.evaluate = si, mi, evm
            parent.indexed_bank = ib
    return pkg
