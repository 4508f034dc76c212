"""Model-level modules of the routed relation path (reference: relation_lm.models)."""
from relation_lm.models.multi_relation_blocks import (
    MultiAnchorRelationBlock,
    MultiRelationBlockConfig,
    RelationBlockStack,
)

__all__ = ["MultiAnchorRelationBlock", "MultiRelationBlockConfig", "RelationBlockStack"]
