"""The C-ABI library loads without a GPU and exports every entry point the
public header declares (no compute calls here)."""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "speculate_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    names = re.findall(r"\b(sd_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_header_declares_the_decoder_surface():
    names = declared_functions()
    for n in ("sd_model_create", "sd_observe", "sd_next_logits", "sd_batched_logits", "sd_rollback_to",
              "sd_tree_logits_keep_kv", "sd_commit_tree_path", "sd_verify_greedy_tree",
              "sd_verify_rejection_linear", "sd_verify_rejection_tree", "sd_set_d2t"):
        assert n in names


def test_library_exports_every_declared_symbol(hip):
    lib = ctypes.CDLL(hip.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
