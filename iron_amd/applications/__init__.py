"""Applications built on the operator library."""
