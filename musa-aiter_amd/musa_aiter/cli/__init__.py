"""Command line interface: ``python -m musa_aiter.cli list-ops`` / ``trace``."""
