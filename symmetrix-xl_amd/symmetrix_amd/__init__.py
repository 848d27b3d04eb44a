"""MI355X-native MACE evaluator (drop-in for the Symmetrix-XL model-evaluation path)."""
