"""The reference's GGUF header fixture, written with the package's GGUF writer."""
from gguf_writer import *  # noqa: F401,F403
from gguf_writer import ARRAY, STR, U32, header


def synth_gguf() -> bytes:
    """The reference's header fixture (gguf.rs:1085-1116): 3 key/values and one tensor-info row,
    no tensor data."""
    return header([("general.architecture", STR, "qwen2moe"), ("general.block_count", U32, 48),
                   ("tokenizer.ggml.tokens", ARRAY, (STR, ["a", "b"]))],
                  [("blk.0.ffn_gate_exps.weight", [2048, 512, 64], 12, 0)])
