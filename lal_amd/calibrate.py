"""Calibration run for hardware byte counters: a plain streaming copy of a known
size (lal_gpu_copy, 16-byte nontemporal loads and stores).

Run under `rocprofv3 --pmc FETCH_SIZE` (then `--pmc WRITE_SIZE`): each
dispatch of copy_f32x4_kernel reads and writes exactly --bytes bytes, so the
counter's reading divided by that size is the factor that turns the same
counter, read on the sampler's dispatches, into HBM bytes.

    python3 -m lal_amd.calibrate --bytes 622854144 --launches 8
"""
import argparse
import json

from lal_amd import abi


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--bytes", type=int, default=1024 * 152064 * 4,
                    help="bytes copied per launch (default: one 1024 x 152064 fp32 batch)")
    ap.add_argument("--launches", type=int, default=8)
    args = ap.parse_args()
    if args.bytes <= 0 or args.bytes % 16:
        raise SystemExit("--bytes must be a positive multiple of 16")
    dev = abi.Device(0, max_batch=1, max_vocab=16)
    src, dst = dev.alloc(args.bytes), dev.alloc(args.bytes)
    abi.check(dev.lib.lal_gpu_synth_uniform(abi.ptr(src), args.bytes // 4, 5, 0.0, 1.0, dev.stream),
              "fill")
    dev.sync()
    e0, e1 = dev.event(), dev.event()
    dev.record(e0)
    for _ in range(args.launches):
        abi.check(dev.lib.lal_gpu_copy(abi.ptr(dst), abi.ptr(src), args.bytes, dev.stream), "copy")
    dev.record(e1)
    dev.sync()
    ms = dev.elapsed_ms(e0, e1) / args.launches
    print(json.dumps({"kernel": "copy_f32x4_kernel", "bytes_read_per_launch": args.bytes,
                      "bytes_written_per_launch": args.bytes, "launches": args.launches,
                      "ms_per_launch": ms, "copy_GBps_read_plus_write": 2 * args.bytes / ms / 1e6}))
    src.close()
    dst.close()
    dev.close()


if __name__ == "__main__":
    main()
