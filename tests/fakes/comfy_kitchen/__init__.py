"""Stand-in for comfy-kitchen (tests only)."""
