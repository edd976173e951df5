"""Test infrastructure: CPU restatement of the reference forward pass (see transformer_oracle)."""
