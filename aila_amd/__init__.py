"""MI355X-native attention hot path for Aila (GQA + Gated DeltaNet)."""
