"""trnblas for AMD MI355X (placeholder; filled in by level3 and dispatch)."""
