"""Placeholder pass (filled in by the WOQ pattern work)."""


def replace_with_zentorch_ops_new(graph):
    return graph
