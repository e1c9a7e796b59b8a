"""argparse namespaces with every precision flag at its default (as the reference's tests build them)."""

from __future__ import annotations

import argparse


def precision_args(**overrides) -> argparse.Namespace:
    from lowbit.precision import add_mixed_precision_args

    parser = argparse.ArgumentParser()
    add_mixed_precision_args(parser)
    ns = parser.parse_args([])
    for k, v in overrides.items():
        setattr(ns, k, v)
    return ns
