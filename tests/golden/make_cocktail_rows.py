"""Write tests/golden/cocktail_rows.npz: generator rows with the metadata the
generator marked while placing each piece (kerneldev_amd.synth.cocktail_batch).

The collate rule (data_builder.py:603-643) assigns is_prefix, in_span and
span_id as it stitches the row together: the prefix and its [CLS], each
[SPAN]..[ES] with id 1 + its placement index, and -1 at [MASKQ].  These rows
carry exactly that construction-time metadata, so the oracle's token-reading
restatement (oracle/metadata.py::collate_metadata) can be checked against it
without importing the product package.  Rows: the config-3 layout (6 rows of
1024, seed 5) and the config-4 layout (2 rows of 8192, seed 0).

    python tests/golden/make_cocktail_rows.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from kerneldev_amd.synth import CONFIG3_LAYOUT, CONFIG4_LAYOUT, cocktail_batch  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cocktail_rows.npz")


def main():
    out = {}
    for name, (B, L, layout, seed) in {"c3": (6, 1024, CONFIG3_LAYOUT, 5), "c4": (2, 8192, CONFIG4_LAYOUT, 0)}.items():
        tokens, in_span, span_id, is_prefix = cocktail_batch(B, L, layout, seed)
        out[f"{name}_tokens"] = tokens.numpy().astype(np.int16)
        out[f"{name}_in_span"] = in_span.numpy()
        out[f"{name}_span_id"] = span_id.numpy().astype(np.int16)
        out[f"{name}_is_prefix"] = is_prefix.numpy()
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
