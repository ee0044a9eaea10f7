#!/usr/bin/env python3
"""Apply the drop-in edits to a copy of
tools/server/qwen7b_server.c:

  1. the include of runtime/lal_sampling.h becomes include/lal_sampling.h
     with LAL_SAMPLING_FILTERED defined;
  2. the server's own lal_sample_token_filtered is removed (the header
     provides it, sampling on the GPU);
  3. after the hot-loaded .lal objects are opened, a loaded lal_filter_topk
     is handed to the header with the server's decode wrapper.

usage: apply_dropin_edits.py SERVER_C OUT_C
The edits are located by one-line anchors; the script fails if an anchor is
not found exactly once, so a changed server source is reported, not patched
silently.
"""
import sys


def edit(src):
    def once(anchor):
        n = src.count(anchor)
        if n != 1:
            raise SystemExit(f"anchor found {n} times: {anchor!r}")
        return src.index(anchor)

    inc = '#include "runtime/lal_sampling.h"\n'
    i = once(inc)
    src = (src[:i] + '#define LAL_SAMPLING_FILTERED 1\n'
           '#include "lal_sampling.h"  /* MI355X sampler (liblal_gpu.so), same API */\n'
           + src[i + len(inc):])
    a = once("static int lal_sample_token_filtered(float *logits, int vocab_size,")
    # back to the start of the comment block just above the function
    c = src.rfind("/*", 0, a)
    b = once("/* === Thread pool for parallel matmul (OpenMP) ===")
    src = (src[:c] + "/* lal_sample_token_filtered: from lal_sampling.h (GPU sampler) */\n\n"
           + src[b:])
    load = 'fprintf(stderr, "[lal] warning: failed to load %s\\n", lal_paths[i]);\n'
    j = once(load) + len(load)
    src = (src[:j] + "    /* the GPU sampler runs a loaded filter through its keep-mask adapter */\n"
           "    if (g_lal_filter) lal_sampling_set_filter_plugin(g_lal_filter, qwen7b_decode_for_filter);\n"
           + src[j:])
    return src


if __name__ == "__main__":
    with open(sys.argv[1], encoding="utf-8") as f:
        out = edit(f.read())
    with open(sys.argv[2], "w", encoding="utf-8") as f:
        f.write(out)
