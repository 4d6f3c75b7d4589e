"""Trainer adapters (torch counterparts of src/mlx_train_perf/adapters/)."""
