"""Parity counts of the GPU tests (flagged tokens, score differences,
admission flips, error maxima): each line is printed when the test makes it
and repeated in pytest's terminal summary, which a quiet (-q) run shows
too."""
LINES = []


def report(line):
    print(line, flush=True)
    LINES.append(line)
