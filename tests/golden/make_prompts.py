"""Writes prompts.npz: the reference's bench prompts as token ids (bench/prompts/*.ids, one
whitespace-separated id list per file), for the prompt-lookup tests.  Data only; run in a
container that holds the reference checkout:  python tests/golden/make_prompts.py"""
import os
import sys

import numpy as np

SRC = "/root/reference/bench/prompts"
NAMES = ["document_6800", "repeat_1800", "running_summary", "message_summary", "tool_json", "alert_text",
         "call_request", "short_command"]


def main():
    out = {}
    for n in NAMES:
        with open(os.path.join(SRC, n + ".ids")) as f:
            out[n] = np.array([int(t) for t in f.read().split()], np.int32)
        print(n, out[n].size)
    np.savez_compressed(os.path.join(os.path.dirname(os.path.abspath(__file__)), "prompts.npz"), **out)


if __name__ == "__main__":
    sys.exit(main())
