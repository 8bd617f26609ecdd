"""Placeholder pass (filled in by the WOQ pattern work)."""


def woq_linear_binary_binary_post_op_fusions(graph):
    return graph
