"""int4 W4A16 for MI355X: int4 weights with bf16 group scales streamed by dense_reader's GEMV."""
