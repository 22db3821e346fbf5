"""Mirror of goda's `mint` attention interfaces backed by the HIP library."""
