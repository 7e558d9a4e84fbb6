"""Writes the block-file fixtures from the reference's committed artifacts (data only):

* block_component_s288.ncnn.param: the reviewed component graph of block 4
  (artifacts/2026-09-05/components/blocks/block-04/runtime/block.ncnn.param),
  288 tokens, BinaryOp residual adds;
* block_runtime_s4160.ncnn.param: the runtime package graph of block 4
  (artifacts/2026-09-05/pipeline/models/dit-s4160-residual-v1/block-04/block.ncnn.param),
  4160 tokens, ErnieResidualAdd;
* block04_sections.json: the ModelBin section table the reference recorded for
  that block's BF16 weight file (layer, tensor shape, storage kind and byte
  range [begin, end) per section, from the same directory's model.json), and
  the graph-contract hash recorded there.
"""
import json
import shutil
from pathlib import Path

REF = Path("/root/reference/artifacts/2026-09-05")
OUT = Path(__file__).resolve().parent

shutil.copyfile(REF / "components/blocks/block-04/runtime/block.ncnn.param", OUT / "block_component_s288.ncnn.param")
shutil.copyfile(REF / "pipeline/models/dit-s4160-residual-v1/block-04/block.ncnn.param",
                OUT / "block_runtime_s4160.ncnn.param")
comp = json.loads((REF / "components/blocks/block-04/runtime/model.json").read_text())
storage = comp["weight_storage"]
table = {
    "source": "artifacts/2026-09-05/components/blocks/block-04/runtime/model.json",
    "tokens": comp["tokens"],
    "graph_contract_sha256": storage["graph_contract_sha256"],
    "sections": [{"layer": s["layer"], "shape": s["shape"], "storage": s["storage"],
                  "begin": s["output_offsets"][0], "end": s["output_offsets"][1]} for s in storage["sections"]],
}
(OUT / "block04_sections.json").write_text(json.dumps(table, indent=1) + "\n")
print(len(table["sections"]), "sections; bin bytes", table["sections"][-1]["end"])
