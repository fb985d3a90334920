"""etx.operators: operator providers of the decode path (reference: etx/operators/)."""
