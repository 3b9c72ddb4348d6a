"""MI355X-native TileInfer decode worker: planner (tileplan), C-ABI binding (runtime) and build."""
