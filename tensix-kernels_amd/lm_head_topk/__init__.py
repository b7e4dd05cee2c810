"""lm_head_topk for MI355X: an LM head that returns token ids, built on dense_reader's top-k records."""
