"""Weight formats of the hot path (kquant/io/)."""
