"""Test-only checkers: the float64 oracle and the CPU port of the reference path.

Nothing in the product package imports this directory.
"""
