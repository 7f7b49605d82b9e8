"""Programs written against the reference's API, as a reference user writes them (the names
resolve to the test double of the reference package)."""

import reference_double as ninetoothed
import reference_double.language as ntl
from reference_double import Symbol

BLOCK_SIZE = Symbol("BLOCK_SIZE", meta=True)


def add_arrangement(lhs, rhs, output, BLOCK_SIZE=BLOCK_SIZE):
    return lhs.tile((BLOCK_SIZE,)), rhs.tile((BLOCK_SIZE,)), output.tile((BLOCK_SIZE,))


def add_application(lhs, rhs, output):
    output = lhs + rhs  # noqa: F841


def softmax_arrangement(input, output, BLOCK_SIZE=ninetoothed.block_size()):
    return input.tile((1, BLOCK_SIZE)), output.tile((1, BLOCK_SIZE))


def _shifted(x):
    return x - ntl.max(x)


def softmax_application(input, output):
    numerator = ntl.exp(_shifted(input))  # a helper of the user's module, itself using ntl
    output = numerator / ntl.sum(numerator)  # noqa: F841
