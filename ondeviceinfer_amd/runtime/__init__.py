"""Weight-name conventions shared by the runtimes and the linear backends."""
