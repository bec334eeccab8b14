"""Benchmark grids (reference: bench/grid.py:5-43).

The values are the reference's, so that result rows of the two builds cover
the same cells.
"""
import itertools

BENCH_GRID = {
    "B": [32, 128, 512, 2048],
    "d": [768, 2048, 4096],
    "F": [2**14, 2**16, 2**18, 2**20, 2**22],
    "k": [16, 32, 64, 128],
    "dtype": ["fp16", "bf16", "fp32"],
}

BENCH_GRID_CPU = {
    "B": [32, 128, 512],
    "d": [768, 2048],
    "F": [2**14, 2**16, 2**18],
    "k": [16, 32, 64],
    "dtype": ["fp32"],
}

RECALL_GRID = {
    "B": [128, 512],
    "d": [2048, 4096],
    "F": [2**16, 2**18, 2**20],
    "k": [32, 64],
    "c_multiplier": [1, 2, 4, 8, 16],
    "dtype": ["bf16"],
}


def iter_grid(grid):
    """Every combination of a grid, as dicts, in key order (last key fastest)."""
    keys = list(grid)
    for combo in itertools.product(*(grid[k] for k in keys)):
        yield dict(zip(keys, combo))


def dry_run_cell(grid):
    """The first cell of a grid (the --dry-run smoke cell)."""
    return next(iter_grid(grid))


def filter_cells(cells, args):
    """Cells whose B, d, F, k and dtype are in the comma lists given on the command line."""
    for cell in cells:
        if any(getattr(args, key, None) and cell[key] not in getattr(args, key)
               for key in ("B", "d", "F", "k", "dtype")):
            continue
        yield cell
