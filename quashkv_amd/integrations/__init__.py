"""Framework integrations (HuggingFace-style cache)."""
