"""Test oracle for the paged KV path (see tvara_oracle.h): test infrastructure only."""
