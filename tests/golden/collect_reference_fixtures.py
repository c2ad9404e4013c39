"""Copy the reference's recorded result files used as known-answer fixtures.

Run in the build container (where the reference checkout is mounted):
    python tests/golden/collect_reference_fixtures.py [/path/to/reference]
Copies data files only (JSON results the reference recorded); no reference
source is copied or executed:
  * results/virtual-addressing-cpu/geometry.json - chunk counts of the three
    2048-of-65536 support sets (pins VirtualKVLayout.selected_chunks and the
    support-set generator of scripts/analyze_virtual_layout.py:11-27);
  * results/vmm-pair12k-shadow/adaptive_stats/plans-rank0{0..3}.json - page
    ownership snapshots with the chunk-aware demotion plans the reference
    computed (pins plan_demote_pages, adaptive_sparse/migration.py:27-54).
"""

import shutil
import sys
from pathlib import Path

FILES = {
    "results/virtual-addressing-cpu/geometry.json": "virtual_addressing_geometry.json",
    **{f"results/vmm-pair12k-shadow/adaptive_stats/plans-rank0{i}.json": f"demotion_plans_rank{i}.json"
       for i in range(4)},
}


def main():
    reference = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    target = Path(__file__).resolve().parent
    for source, name in FILES.items():
        shutil.copyfile(reference / source, target / name)
        print(f"{source} -> tests/golden/{name}")


if __name__ == "__main__":
    main()
