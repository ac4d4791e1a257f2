"""CPU oracle of the WKV-7 + .rwkvq hot path (test infrastructure only)."""
