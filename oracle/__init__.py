"""CPU oracle of the MoE path — test infrastructure only (see moe_oracle)."""
