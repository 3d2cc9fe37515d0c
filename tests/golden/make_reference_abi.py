"""Writes tests/golden/reference_abi.json: the names and argument kinds of the reference's kernel-library symbols
this library replaces, read as text from the reference's FFI declarations (nothing of the reference is built, imported
or run):
  crates/inference-quant/src/gguf/ffi.rs   the kernel_library! blocks of libinferencequant and libinferencequant_<t>
  crates/inference-nn/src/cuda/ffi.rs      moe_router_topk_{f32,bf16,f16}
The per-type blocks are macro templates (gguf_type_library!, gguf_mmq_type_library!, gguf_standard_type!,
gguf_iq_types!, ffi.rs:835-1290); they are expanded here for the weight types this library serves.  The shared
symbols are kept when they name one of those types or none.  Not kept: the LoRA MoE decode pairs
(moe_lora_decode_kernels!, ffi.rs:11-52, 780-831), the iq4_ks tile entries and the types this library does not
serve.  Run once with the reference checked out at REF; the JSON is the fixture tests/test_abi.py reads.
"""
import json
import os
import re
import sys

REF = os.environ.get("REF", "/root/reference")
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_abi.json")

STANDARD = ["q4_0", "q5_0", "q8_0", "q4_k", "q5_k", "q6_k"]  # gguf_standard_types! members served here
IQ = ["iq4_xs"]                                              # gguf_iq_types! members served here
TC = ["q4_k", "q6_k"]                                        # `tc` standard types
EXACT = ["q8_0"]                                             # `exact` standard types
# the reference's short names in the shared blocks (indexed MoE, fused MoE decode)
SHORT = {"q4_0": "q4_0", "q5_0": "q5_0", "q8_0": "q8_0", "q4_k": "q4k", "q5_k": "q5k", "q6_k": "q6k"}
UNSERVED = ["q2k", "q3k", "q4_1", "q5_1", "q8_1_q8_1", "q2_k", "q3_k", "iq4_ks", "iq4_nl", "iq1_m", "lora", "gate_up_pair"]


def kind(rust_type: str) -> str:
    t = rust_type.strip()
    if t.startswith("*"):
        return "ptr"
    return {"i32": "i32", "u32": "u32", "i64": "i64", "f32": "f32", "bool": "bool"}[t]


FN = re.compile(r"pub fn\s+(\[<[^>]*>\]|\w+)\s*\(([^)]*)\)\s*(->\s*(\w+))?\s*;", re.S)


def parse(text: str):
    for m in FN.finditer(text):
        name, args, ret = m.group(1), m.group(2), m.group(4)
        kinds = [kind(a.split(":", 1)[1]) for a in args.split(",") if ":" in a]
        yield name, kinds, ret or "void"


def template_name(name: str, t: str) -> str:
    # [<launch_mmvq_gguf_ $t _bf16_plain>] -> launch_mmvq_gguf_q4_k_bf16_plain
    inner = name[2:-2].split()
    return "".join(t if p == "$t" else p for p in inner)


def main() -> None:
    gguf = open(os.path.join(REF, "crates/inference-quant/src/gguf/ffi.rs")).read()
    nn = open(os.path.join(REF, "crates/inference-nn/src/cuda/ffi.rs")).read()
    out = {}
    for name, kinds, ret in parse(gguf):
        if name.startswith("[<"):
            if "launch_mmvq_tc_gguf_" in name:
                types = TC
            elif "_exact>" in name:
                types = EXACT
            elif "launch_dequantize_" in name:
                types = IQ
            elif "fused_glu" in name or "fused_qkv" in name:
                types = STANDARD
            elif "iq4_ks" in name or "untile" in name or "_tiled" in name:  # gguf_iq_tc_types! (not served)
                types = []
            else:  # the matvec, MoE and MMQ entries every served type has
                types = STANDARD + IQ
            for t in types:
                out[template_name(name, t)] = {"args": kinds, "ret": ret}
        else:
            if any(u in name for u in UNSERVED):
                continue
            if "indexed_moe_forward" in name or "moe_gemv" in name:
                if not any(f"_{s}_q8_1" in name for s in SHORT.values()):
                    continue
            out[name] = {"args": kinds, "ret": ret}
    for name, kinds, ret in parse(nn):
        if name.startswith("moe_router_topk_"):
            out[name] = {"args": kinds, "ret": ret}
    json.dump(dict(sorted(out.items())), open(OUT, "w"), indent=0)
    print(f"{len(out)} symbols -> {OUT}", file=sys.stderr)


if __name__ == "__main__":
    main()
