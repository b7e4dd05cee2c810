"""MoE for MI355X: a mixture-of-experts layer that streams only the chosen experts' bfloat4_b weights (moe8)."""
