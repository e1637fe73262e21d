"""Scaled-FP8 paged KV ops (store, paged decode, compaction) on MI355X."""
