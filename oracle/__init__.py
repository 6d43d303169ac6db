"""CPU oracle of the streamed attention path (test infrastructure only)."""
