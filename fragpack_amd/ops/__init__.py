"""GPU KV store and fused attention operators (reference: fragpack/ops)."""
