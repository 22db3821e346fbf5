"""Mirror of goda's `mint.nn` attention and `mint.kvcache` interfaces backed
by the HIP library (same class names, signatures and results)."""
