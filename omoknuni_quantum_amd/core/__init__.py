"""Search API (MCTS, MCTSConfig) and the device wave engine."""
