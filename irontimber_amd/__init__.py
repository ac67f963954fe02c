"""irontimber_amd: MI355X (gfx950) attention / Gated-DeltaNet hot path of the IronTimber engine.

The compute lives in lib/libit_attn.so (hand-written HIP, C ABI in include/it_attn.h); this
package only binds it (`_lib`), offers torch-tensor wrappers (`ops`) and seeded workload
generators (`synth`).
"""
import os

ROOT = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(ROOT, "lib")
