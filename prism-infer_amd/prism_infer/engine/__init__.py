"""Host-side contracts of the KV path (format constants, compaction slot plans)."""
