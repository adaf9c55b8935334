"""Operator wrappers with the reference's Python signatures (``flashrec.kernel``).

As the reference package does (python/flashrec/kernel/__init__.py), the
beam-search entry points are re-exported here."""

from flashrec_amd.kernel.beam_trie import (  # noqa: F401
    GenrecFusedResult,
    GenrecFusedWorkspace,
    beam_expand_token_ids,
    genrec_mask_topk_expand,
    trie_advance_nodes,
    trie_mask_candidates,
    try_load_beam_trie,
)

__all__ = [
    "GenrecFusedResult",
    "GenrecFusedWorkspace",
    "beam_expand_token_ids",
    "genrec_mask_topk_expand",
    "trie_advance_nodes",
    "trie_mask_candidates",
    "try_load_beam_trie",
]
