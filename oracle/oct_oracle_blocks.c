void oct_oracle_blocks_placeholder(void) {}
