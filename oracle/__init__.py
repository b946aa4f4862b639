"""Oracle package: test infrastructure only (see binding.py)."""
