"""Writes tests/golden/v1_random_actions.npz: the random half of the action stream of the
reference's v1 parity run (gpu-d1/scripts/test_learning.py:39-48). That run seeds torch's
global CPU generator once (torch.manual_seed(137)), then for 1, 6 and 8 enemies steps 37
worlds 300 times, taking torch.randint(0, 9, (37,)) on odd steps and the pursuit controller's
actions on even ones (nothing else in the run draws from the generator). The array holds the
odd steps' draws in that order: [3 runs, 150 odd steps, 37 worlds], values 0-8.

Run from the repository root: python tests/golden/make_v1_actions.py
"""
import pathlib

import numpy as np
import torch

OUT = pathlib.Path(__file__).resolve().parent / 'v1_random_actions.npz'


def main():
    torch.manual_seed(137)
    draws = np.zeros((3, 150, 37), np.uint8)
    for run in range(3):
        for k in range(300):
            if k % 2:
                draws[run, k // 2] = torch.randint(0, 9, (37,)).numpy()
    np.savez_compressed(OUT, actions=draws)
    print(f'wrote {OUT} ({draws.size} actions)')


if __name__ == '__main__':
    main()
