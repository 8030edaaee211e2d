"""CPU oracle (test infrastructure only): float64 restatement of the reference's
dequantise-then-attend decode path. Never imported by the operator itself."""
