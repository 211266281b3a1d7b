"""Op contracts: shapes, case lists, seeded input generators and PyTorch standard ops: the reference's three ops and
this build's single-token decode (contiguous and paged) and paged shared-prefix decode."""
from . import prefix, prefix_paged, spec, dsa, decode, decode_paged  # noqa: F401
from . import dsa_project  # noqa: F401  (DSA's input projections; not a verifier op)

OPS = {"prefix": prefix, "prefix_paged": prefix_paged, "spec": spec, "dsa": dsa, "decode": decode,
       "decode_paged": decode_paged}

# Inputs each op's kernel receives (keyword arguments; optional ones absent from the inputs arrive as None).
# The reference's lists (verify.py:35-37) plus this build's optional ragged-suffix lengths for prefix.
KEYS = {"prefix": ["q", "kp", "vp", "ks", "vs", "slens"],
        "spec": ["q", "k", "v", "bits"],
        "dsa": ["q", "kv", "iq", "ik", "w", "lens"],
        "decode": ["q", "k", "v", "lens"],
        "prefix_paged": ["q", "k_pages", "v_pages", "prefix_pages", "suffix_pages", "slens", "layout"],
        "decode_paged": ["q", "k_pages", "v_pages", "page_table", "lens", "layout"]}


def load_op(name):
    return OPS[name]
