"""Writes gen_check.json: check values of the seeded input generator, produced by
this build's own C oracle (oracle/wave_attn_oracle.c) -- NOT by the reference,
which has no normal sampler and was never run.  They freeze the stream that
every benchmark and parity test draws from (xorshift64 as src/common/rng.rs:24-34,
Box-Muller as defined in oracle/wave_attn_oracle.c)."""
import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))
import oracle  # noqa: E402


def main():
    out = {"_source": __doc__.strip(), "cases": []}
    for seed in (42, 1, 0x9E3779B97F4A7C15):
        r = oracle.Xorshift64(seed)
        u64 = [r.next_u64() for _ in range(8)]
        r = oracle.Xorshift64(seed)
        f32 = [r.next_f32() for _ in range(8)]
        r = oracle.Xorshift64(seed)
        normal = [float(x) for x in r.normal(9, 1.0)]
        out["cases"].append({"seed": seed, "next_u64": [str(x) for x in u64],
                             "next_f32": f32, "normal_stddev1": normal,
                             "state_after_9_normals": str(r.state.value)})
    (HERE / "gen_check.json").write_text(json.dumps(out, indent=1) + "\n")


if __name__ == "__main__":
    main()
