"""Puts the h3mi package (two directories above this node, or $H3MI_HOME) on sys.path."""
import os
import sys


def ensure():
    home = os.environ.get("H3MI_HOME") or os.path.dirname(os.path.dirname(os.path.dirname(os.path.realpath(__file__))))
    if home not in sys.path:
        sys.path.insert(0, home)
    return home
