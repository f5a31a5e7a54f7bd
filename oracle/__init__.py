"""TEST INFRASTRUCTURE ONLY: CPU restatements of the reference TCQ quantizer (the checker, never the product)."""
