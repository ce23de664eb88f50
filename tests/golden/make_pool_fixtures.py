"""Write the pooling fixtures from the reference's own golden files.

Reads reference/goldens/{minilm_l6,bge-base-en-v1.5_l12}_s64_boundary.npz (HF
fp32 outputs of the real checkpoints, batch 4, seq 64) with numpy's safe
loader and keeps only what pins app::pool_rows (app_state.hpp:335-374):

  minilm_s64_pool.npz   input_ids, attention_mask, last_hidden_state (full),
                        pool_mean (hf.pool.mean), embedding (hf.out.embedding)
  bge_base_s64_cls.npz  input_ids, attention_mask, last_hidden_state rows 0..3
                        of each sequence, embedding (hf.out.embedding),
                        st_embedding (st.embedding)

Data only: the arrays are copied out of the .npz as they are.
Run in the build container: python tests/golden/make_pool_fixtures.py
"""
import os
import sys

import numpy as np

SRC = "/root/reference/reference/goldens"
DST = os.path.dirname(os.path.abspath(__file__))


def main():
    z = np.load(os.path.join(SRC, "minilm_l6_s64_boundary.npz"), allow_pickle=False)
    np.savez_compressed(
        os.path.join(DST, "minilm_s64_pool.npz"),
        input_ids=z["input_ids"].astype(np.int32),
        attention_mask=z["attention_mask"].astype(np.float32),
        last_hidden_state=z["hf.last_hidden_state"],
        pool_mean=z["hf.pool.mean"],
        embedding=z["hf.out.embedding"],
    )
    z = np.load(os.path.join(SRC, "bge-base-en-v1.5_l12_s64_boundary.npz"), allow_pickle=False)
    np.savez_compressed(
        os.path.join(DST, "bge_base_s64_cls.npz"),
        input_ids=z["input_ids"].astype(np.int32),
        attention_mask=z["attention_mask"].astype(np.float32),
        last_hidden_state_head=z["hf.last_hidden_state"][:, :4, :],
        embedding=z["hf.out.embedding"],
        st_embedding=z["st.embedding"],
    )
    return 0


if __name__ == "__main__":
    sys.exit(main())
