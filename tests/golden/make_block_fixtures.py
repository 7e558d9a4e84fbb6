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
  the graph-contract hash recorded there;
* block00_runtime_fixture.json: the reference's fixture record of block 0
  (artifacts/2026-09-05/components/blocks/block-00/runtime/fixture.json): token
  and grid layout, and the SHA-256 of each official input tensor in0..in9 (in7/in8
  are the official position embeddings, in9 the dense attention mask), copied as is;
* head_{input,output}_s288.ncnn.param: the DiT head graphs of the component export
  (artifacts/2026-09-05/components/heads/{input,output}/head.ncnn.param, 4x4 latent grid
  + 272 text slots) and head_{input,output}_s4160.ncnn.param, the runtime package's
  (artifacts/2026-09-05/pipeline/models/dit-heads-s4160-v1, 64x64 grid + 64 text slots);
  heads.json records the graph SHA-256 each directory's model.json lists for them;
* text_s64.ncnn.param: the reference's 64-token Mistral text block graph
  (tests/fixtures/text-s64.ncnn.param); text_block04_sections.json: the ModelBin
  section table recorded for text block 4
  (artifacts/2026-09-05/pipeline/models/text-s32-v2/block-04/model.json: layer, shape
  and storage per section, in .bin order).
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
shutil.copyfile(REF / "components/blocks/block-00/runtime/fixture.json", OUT / "block00_runtime_fixture.json")
heads = {}
for kind in ("input", "output"):
    for tag, directory in (("s288", REF / "components/heads" / kind),
                           ("s4160", REF / "pipeline/models/dit-heads-s4160-v1" / kind)):
        name = f"head_{kind}_{tag}.ncnn.param"
        shutil.copyfile(directory / "head.ncnn.param", OUT / name)
        heads[name] = json.loads((directory / "model.json").read_text())["files"]["head.ncnn.param"]
(OUT / "heads.json").write_text(json.dumps(heads, indent=1) + "\n")
shutil.copyfile(REF.parent / "../tests/fixtures/text-s64.ncnn.param", OUT / "text_s64.ncnn.param")
text = json.loads((REF / "pipeline/models/text-s32-v2/block-04/model.json").read_text())
(OUT / "text_block04_sections.json").write_text(json.dumps({
    "source": "artifacts/2026-09-05/pipeline/models/text-s32-v2/block-04/model.json",
    "tokens": text["tokens"], "graph_sha256": text["graph_sha256"],
    "sections": [{"layer": s["layer"], "shape": s["shape"], "storage": s["storage"]} for s in text["sections"]],
}, indent=1) + "\n")
print(len(table["sections"]), "sections; bin bytes", table["sections"][-1]["end"])
