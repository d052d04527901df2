"""Golden fixtures of the pooling path (data only) and the script that writes them."""
