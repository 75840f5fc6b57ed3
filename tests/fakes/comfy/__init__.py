"""Stand-in for ComfyUI's comfy package (tests only)."""
