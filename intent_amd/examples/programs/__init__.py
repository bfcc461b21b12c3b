"""Multi-kernel example programs (the reference's `python/intent/examples/programs/`)."""
