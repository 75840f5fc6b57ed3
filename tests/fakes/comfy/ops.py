"""Stand-in for comfy.ops (tests only): the per-op hook counter."""
RUN_EVERY_OP_CALLS = [0]


def run_every_op():
    RUN_EVERY_OP_CALLS[0] += 1
