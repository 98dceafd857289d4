"""Runtime backends. Only the single-process (world_size=1) backend exists in this build."""
