"""aiter integration: the ``provider`` package answers aiter's routed-op calls."""
