"""CPU oracle (test infrastructure only): a C restatement of Mantle's CPU decode path."""
