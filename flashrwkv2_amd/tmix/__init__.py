"""TMix operators of flashrwkv2_amd (the WKV7 recurrence)."""
