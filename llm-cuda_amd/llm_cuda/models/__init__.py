"""Model package."""
