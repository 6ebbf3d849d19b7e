"""Copy the reference's checkpoint-header fixtures (data only: the real 27B checkpoint's config.json and the dtype and
shape of each of its 1,616 tensors, which the reference's tests/test_real_checkpoint.py reads) into tests/golden/.

    python tests/golden/copy_checkpoint_header.py /root/reference
"""

import shutil
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent


def main(reference: str) -> None:
    src = Path(reference) / "tests" / "fixtures"
    shutil.copyfile(src / "config.json", HERE / "ref_27b_config.json")
    shutil.copyfile(src / "model.header.json", HERE / "ref_27b_model.header.json")
    print("copied", src / "config.json", src / "model.header.json")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
