#!/usr/bin/env python3
"""Export a local HuggingFace Qwen3 checkpoint to the decoder's on-disk format.

Command-line counterpart of examples/qwen3_asr/export_weights.py in the
reference, on top of matmul_decoder_export_hf_model (csrc/host/md_export.c):

    python export_weights.py --model /path/to/hf_checkpoint --output-dir ./qwen3-matmul \\
        [--quant fp16|int8|int4]

The checkpoint directory holds config.json and one or more *.safetensors
files (F32, F16 or BF16).  Output: config.json, embeddings.bin, lm_head.bin
when the head is untied, final_norm.bin and layer_LL/ with the fp32 norms and
the projections as fp16 [K,N] (fp16) or <proj>_weight.bin + <proj>_scales.bin
(int8, int4).  Models are read from disk only; nothing is downloaded.
"""
import argparse
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import mdx_lib  # noqa: E402


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--model", required=True, help="local HuggingFace checkpoint directory")
    ap.add_argument("--output-dir", required=True, help="output directory")
    ap.add_argument("--quant", default="fp16", choices=["fp16", "int8", "int4"],
                    help="projection format (default fp16)")
    args = ap.parse_args(argv)
    if not os.path.isdir(args.model):
        print(f"export_weights.py: {args.model} is not a directory", file=sys.stderr)
        return 1
    mdx_lib.export_hf_model(args.model, args.output_dir, args.quant)
    print(f"exported {args.model} -> {args.output_dir} ({args.quant})")
    return 0


if __name__ == "__main__":
    sys.exit(main())
