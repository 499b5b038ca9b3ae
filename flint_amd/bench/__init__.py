"""flint_bench support: the JSON log renderer (results_table)."""
