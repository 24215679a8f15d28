"""Lowering of online-softmax attention loop nests (placeholder until written)."""
def match(plan):
    return None
def lower(*a, **k):
    raise NotImplementedError
