"""CDNAv3 directory -> one HF-loadable safetensors file (+ config.json).

Same key convention and entry points as the reference
(``helix_substrate/convert_safetensors.py:1-26`` naming, ``:53-96``
per-tensor loading, ``:156-235`` conversion, ``:238-269`` the
quantization_config, ``:272-347`` the directory conversion):

    {module}.codebook            [k] fp32
    {module}.indices             [out, in / vector_dim] uint8 (int16 when the
                                  directory's index_dtype is "uint16")
    {module}.sidecar_positions   [n] int64     (optional)
    {module}.sidecar_values      [n] fp32      (optional)
    {module}.svd_U / svd_s / svd_Vt, {module}.channel_scales (optional)
    {module}.group_scale / group_offset [out, in/G] fp32 (the affine
                                  extension; meta "group_size")

Exact tensors (``*.npy`` + ``*.npy.meta.json``) keep their names; tensors the
compressor never exported (e.g. Mamba's A_log, D) can be pulled from the
original checkpoint.  ``HelixHfQuantizer`` (hf_quantizer.py) loads the result
back into ``HelixLinear`` modules.
"""
from __future__ import annotations

import json
import shutil
import time
from pathlib import Path
from typing import Dict, Optional

import numpy as np

_TOKENIZER_FILES = ("tokenizer.json", "tokenizer_config.json", "tokenizer.model",
                    "special_tokens_map.json", "added_tokens.json", "generation_config.json")


def _module_base(tensor_name: str) -> str:
    return tensor_name[:-7] if tensor_name.endswith(".weight") else tensor_name


def _load_cdnav3_tensors(tensor_dir) -> Dict[str, np.ndarray]:
    """Every component of one ``.cdnav3`` directory under its safetensors key."""
    tensor_dir = Path(tensor_dir)
    meta = json.loads((tensor_dir / "meta.json").read_text())
    rows, cols = meta["shape"]
    base = _module_base(meta["tensor_name"])
    wide = meta.get("index_dtype", "uint8") == "uint16"
    idx = np.fromfile(tensor_dir / "indices.bin", dtype=np.uint16 if wide else np.uint8)
    idx = idx.reshape(rows, cols // int(meta.get("vector_dim", 1)))
    out = {
        f"{base}.codebook": np.load(tensor_dir / "codebook.npy").astype(np.float32),
        # torch has no uint16: wide indices travel as int16 (all below 4096)
        f"{base}.indices": idx.astype(np.int16) if wide else idx,
    }
    sc = tensor_dir / "sidecar.npz"
    if sc.exists():
        with np.load(sc, allow_pickle=False) as z:
            if "positions" in z and z["positions"].size > 0:
                out[f"{base}.sidecar_positions"] = z["positions"].astype(np.int64)
                out[f"{base}.sidecar_values"] = z["values"].astype(np.float32)
    optional = ("svd_U", "svd_s", "svd_Vt", "channel_scales", "group_scale", "group_offset")
    for name in optional:
        f = tensor_dir / f"{name}.npy"
        if f.exists():
            out[f"{base}.{name}"] = np.load(f, allow_pickle=False).astype(np.float32)
    return out


def _load_exact_tensor(npy_path) -> tuple:
    """(name, array) of an exact tensor; the name comes from its companion
    ``.npy.meta.json`` (else the file stem with '_' -> '.')."""
    npy_path = Path(npy_path)
    meta_path = npy_path.parent / f"{npy_path.name}.meta.json"
    if meta_path.exists():
        name = json.loads(meta_path.read_text()).get("tensor_name", npy_path.stem)
    else:
        name = npy_path.stem.replace("_", ".")
    return name, np.load(npy_path, allow_pickle=False)


def _load_missing_from_original(all_tensors: dict, original_safetensors,
                                compressed_modules) -> int:
    """Add the original checkpoint's tensors that the CDNAv3 export lacks
    (skipping the dense weights of compressed modules); returns the count."""
    from safetensors import safe_open

    skip = {f"{m}.weight" for m in compressed_modules}
    added = 0
    with safe_open(str(original_safetensors), framework="pt") as f:
        for key in f.keys():
            if key in all_tensors or key in skip:
                continue
            all_tensors[key] = f.get_tensor(key).float().numpy()
            added += 1
    return added


def convert_cdnav3_to_safetensors(cdnav3_dir, output_path, original_model_path=None) -> dict:
    """All ``*.cdnav3`` dirs and exact ``*.npy`` tensors of a CDNAv3 output
    directory -> one safetensors file; returns conversion stats."""
    from safetensors.numpy import save_file

    cdnav3_dir, output_path = Path(cdnav3_dir), Path(output_path)
    tensors: Dict[str, np.ndarray] = {}
    compressed, group_sizes = [], set()
    k_map, vd_map = {}, {}
    n_exact = 0
    for d in sorted(cdnav3_dir.glob("*.cdnav3")):
        meta_path = d / "meta.json"
        if not d.is_dir() or not meta_path.exists():
            continue
        meta = json.loads(meta_path.read_text())
        if meta.get("storage_mode") == "exact":
            continue
        tensors.update(_load_cdnav3_tensors(d))
        base = _module_base(meta["tensor_name"])
        compressed.append(base)
        k = int(np.load(d / "codebook.npy", mmap_mode="r").shape[0])
        if k != 256:  # the loader's shells need the codebook size and index width
            k_map[base] = k
        if int(meta.get("vector_dim", 1)) != 1:
            vd_map[base] = int(meta["vector_dim"])
        if "group_size" in meta and (d / "group_scale.npy").exists():
            group_sizes.add(int(meta["group_size"]))
    for f in sorted(cdnav3_dir.glob("*.npy")):
        name, arr = _load_exact_tensor(f)
        tensors[name] = arr.astype(np.float32)
        n_exact += 1
    n_orig = 0
    if original_model_path is not None and Path(original_model_path).exists():
        n_orig = _load_missing_from_original(tensors, original_model_path, compressed)
    if len(group_sizes) > 1:
        raise ValueError(f"mixed affine group sizes {sorted(group_sizes)} are not supported")
    output_path.parent.mkdir(parents=True, exist_ok=True)
    save_file({k: np.ascontiguousarray(v) for k, v in tensors.items()}, str(output_path))
    size = output_path.stat().st_size
    return {"n_compressed": len(compressed), "n_exact": n_exact, "n_from_original": n_orig,
            "n_total_keys": len(tensors), "output_bytes": size,
            "output_mb": round(size / 1024 / 1024, 1), "compressed_modules": compressed,
            "group_size": next(iter(group_sizes)) if group_sizes else None,
            "module_k_map": k_map, "module_vector_dim_map": vd_map}


def write_quantization_config(model_config_path, output_config_path, compressed_modules,
                              manifest: Optional[dict] = None, group_size=None,
                              module_k_map=None, module_vector_dim_map=None) -> None:
    """config.json + ``quantization_config`` (quant_method "cdna_v3")."""
    config = json.loads(Path(model_config_path).read_text())
    q = {"quant_method": "cdna_v3", "bits": 8, "n_clusters": 256,
         "compressed_modules": list(compressed_modules)}
    if manifest:
        q["compression_ratio"] = manifest.get("compression_ratio", 4.0)
        q["n_svd_routed"] = manifest.get("n_svd_routed", 0)
    if group_size:
        q["group_size"] = int(group_size)
    if module_k_map:
        q["module_k_map"] = dict(module_k_map)
    if module_vector_dim_map:
        q["module_vector_dim_map"] = dict(module_vector_dim_map)
    config["quantization_config"] = q
    out = Path(output_config_path)
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text(json.dumps(config, indent=2) + "\n")


def convert_model(cdnav3_dir, model_dir, output_dir) -> dict:
    """CDNAv3 dir + original HF model dir -> HF directory (model.safetensors,
    config.json with quantization_config, tokenizer files, manifest copy,
    conversion_receipt.json)."""
    cdnav3_dir, model_dir, output_dir = Path(cdnav3_dir), Path(model_dir), Path(output_dir)
    output_dir.mkdir(parents=True, exist_ok=True)
    t0 = time.time()
    original = None
    for cand in (model_dir / "model.safetensors", model_dir / "model-00001-of-00001.safetensors"):
        if cand.exists():
            original = cand
            break
    if original is None:
        shards = sorted(model_dir.glob("model-*.safetensors"))
        original = shards[0] if shards else None
    stats = convert_cdnav3_to_safetensors(cdnav3_dir, output_dir / "model.safetensors", original)
    manifest = {}
    if (cdnav3_dir / "manifest.json").exists():
        manifest = json.loads((cdnav3_dir / "manifest.json").read_text())
    if (model_dir / "config.json").exists():
        write_quantization_config(model_dir / "config.json", output_dir / "config.json",
                                  stats["compressed_modules"], manifest, stats["group_size"],
                                  stats["module_k_map"], stats["module_vector_dim_map"])
    for name in _TOKENIZER_FILES:
        if (model_dir / name).exists():
            shutil.copy2(model_dir / name, output_dir / name)
    if (cdnav3_dir / "manifest.json").exists():
        shutil.copy2(cdnav3_dir / "manifest.json", output_dir / "cdnav3_manifest.json")
    stats["wall_time_s"] = round(time.time() - t0, 2)
    stats["output_dir"] = str(output_dir)
    (output_dir / "conversion_receipt.json").write_text(json.dumps(stats, indent=2) + "\n")
    return stats
