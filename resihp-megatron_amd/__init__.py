"""MI355X-native MoE expert-parallel layer hot path (placeholder during bring-up)."""
