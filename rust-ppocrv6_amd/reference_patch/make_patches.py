"""Writes the executor and pipeline edits of the HIP head as unified diffs against the
reference crate: patches/engine_model.patch (src/engine/model.rs) and patches/pipeline.patch
(src/pipeline.rs).  The edits are applied to scratch copies of the two files (outside this
repository) and only the diffs are kept; apply them in the reference crate with
`patch -p1 < patches/<name>.patch`, together with the files under src/ here
(src/ops/gpu_head.rs, src/ops/gpu_neck.rs, src/postprocess/ctc/gpu.rs).

    python make_patches.py /path/to/rust-ppocrv6
"""
import os
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))


def edit(text, old, new, count=1):
    assert text.count(old) == count, (old[:80], text.count(old))
    return text.replace(old, new)


def model_rs(s):
    s = edit(s, "use crate::ops::{self, Conv2dParams, ConvTranspose2dParams, Pool2dParams};\n",
             "use crate::ops::gpu_head::{GpuHead, RecHeadBackend};\n"
             "use crate::ops::{self, Conv2dParams, ConvTranspose2dParams, Pool2dParams};\n")
    s = edit(s, "    quantized_matmul_weights: HashMap<String, ops::QuantizedWeight>,\n}\n",
             "    quantized_matmul_weights: HashMap<String, ops::QuantizedWeight>,\n"
             "    /// HIP heads by MatMul node name (attach_gpu_heads).\n"
             "    gpu_heads: HashMap<String, GpuHead>,\n"
             "    /// Outputs of those MatMuls whose one use is a Softmax graph output, with the\n"
             "    /// Softmax's axis: the head writes them as probabilities (one call, no logits).\n"
             "    fused_softmax: HashMap<String, isize>,\n}\n")
    s = edit(s, "            transposed_matmul_weights,\n            quantized_matmul_weights,\n        })\n",
             "            transposed_matmul_weights,\n            quantized_matmul_weights,\n"
             "            gpu_heads: HashMap::new(),\n            fused_softmax: HashMap::new(),\n        })\n")
    s = edit(s, "    /// Whether any MatMul weights are quantized in this model.\n",
             "    /// With `RecHeadBackend::Hip`, a HIP head for every MatMul whose weight was prepacked:\n"
             "    /// the INT8 head from its QuantizedWeight (after quantize_matmul_weights) or the FP32\n"
             "    /// head from W^T, with the MatMul's folded bias; and the segments MatMul -> Softmax ->\n"
             "    /// graph output the head runs as one call.  The host weights stay, so\n"
             "    /// weight_footprint_bytes is unchanged.  Nothing changes on an error.\n"
             "    pub fn attach_gpu_heads(&mut self, backend: RecHeadBackend) -> Result<()> {\n"
             "        let mut heads = HashMap::new();\n"
             "        if let RecHeadBackend::Hip { device } = backend {\n"
             "            for node in self.graph.nodes.iter().filter(|n| n.op == \"MatMul\" && n.inputs.len() >= 2) {\n"
             "                let w = &node.inputs[1];\n"
             "                let bias = node.inputs.get(2).filter(|b| !b.is_empty()).and_then(|b| self.weights.get(b));\n"
             "                let head = if let Some(qw) = self.quantized_matmul_weights.get(w) {\n"
             "                    GpuHead::new(qw, bias, device)?\n"
             "                } else if let Some(w_t) = self.transposed_matmul_weights.get(w) {\n"
             "                    GpuHead::new_f32(w_t, bias, device)?\n"
             "                } else {\n"
             "                    continue;\n"
             "                };\n"
             "                heads.insert(node.name.clone(), head);\n"
             "            }\n"
             "        }\n"
             "        let outputs: HashSet<&str> = self.graph.outputs.iter().map(|o| o.as_str()).collect();\n"
             "        let head_outs: HashSet<&str> = self.graph.nodes.iter()\n"
             "            .filter(|n| heads.contains_key(&n.name)).map(|n| n.outputs[0].as_str()).collect();\n"
             "        let mut fused = HashMap::new();\n"
             "        for node in self.graph.nodes.iter().filter(|n| n.op == \"Softmax\") {\n"
             "            let x = node.inputs[0].as_str();\n"
             "            if outputs.contains(node.outputs[0].as_str()) && head_outs.contains(x)\n"
             "                && self.usage_counts.get(x) == Some(&1) {\n"
             "                let axis = node.attrs.get(\"axis\").and_then(|a| a.as_i64()).unwrap_or(-1) as isize;\n"
             "                fused.insert(x.to_string(), axis);\n"
             "            }\n"
             "        }\n"
             "        self.gpu_heads = heads;\n"
             "        self.fused_softmax = fused;\n"
             "        Ok(())\n"
             "    }\n\n"
             "    /// The HIP head of the fused segment and the name of the tensor it reads, for callers\n"
             "    /// that batch text lines (OcrEngine::recognize).\n"
             "    pub fn rec_head(&self) -> Option<(&GpuHead, &str)> {\n"
             "        self.graph.nodes.iter().find_map(|n| {\n"
             "            let head = self.gpu_heads.get(&n.name)?;\n"
             "            self.fused_softmax.contains_key(&n.outputs[0]).then(|| (head, n.inputs[0].as_str()))\n"
             "        })\n"
             "    }\n\n"
             "    /// Whether any MatMul weights are quantized in this model.\n")
    s = edit(s, "    pub fn forward(&self, input_name: &str, input_tensor: Tensor) -> Result<Tensor> {\n"
                "        let (out, _) = self.forward_internal(input_name, input_tensor, false)?;\n"
                "        Ok(out)\n    }\n",
             "    pub fn forward(&self, input_name: &str, input_tensor: Tensor) -> Result<Tensor> {\n"
             "        let (out, _) = self.forward_internal(input_name, input_tensor, false, None)?;\n"
             "        Ok(out)\n    }\n\n"
             "    /// forward() up to the tensor named `stop`, which it returns (e.g. the head's input).\n"
             "    pub fn forward_until(&self, input_name: &str, input_tensor: Tensor, stop: &str) -> Result<Tensor> {\n"
             "        let (out, _) = self.forward_internal(input_name, input_tensor, false, Some(stop))?;\n"
             "        Ok(out)\n    }\n")
    s = edit(s, "        self.forward_internal(input_name, input_tensor, true)\n",
             "        self.forward_internal(input_name, input_tensor, true, None)\n")
    s = edit(s, "        input_tensor: Tensor,\n        profile: bool,\n    ) -> Result<(Tensor, HashMap<String, f64>)> {\n",
             "        input_tensor: Tensor,\n        profile: bool,\n        stop: Option<&str>,\n"
             "    ) -> Result<(Tensor, HashMap<String, f64>)> {\n"
             "        if stop == Some(input_name) {\n"
             "            return Ok((input_tensor, HashMap::new()));\n"
             "        }\n")
    s = edit(s, "                    if let Some(qw) = self.quantized_matmul_weights.get(w_name) {\n"
                "                        ops::matmul_quantized_b(a, qw, bias)?\n",
             "                    if let Some(head) = self.gpu_heads.get(&node.name) {\n"
             "                        // the fused segment: probabilities straight from the projection\n"
             "                        match self.fused_softmax.get(out_name.as_str()) {\n"
             "                            Some(&axis) if softmax_axis_is_last(axis, a.shape().len()) => head.probs(a)?,\n"
             "                            _ => head.logits(a)?,\n"
             "                        }\n"
             "                    } else if let Some(qw) = self.quantized_matmul_weights.get(w_name) {\n"
             "                        ops::matmul_quantized_b(a, qw, bias)?\n")
    s = edit(s, "                    if usage_count.get(in_name) == Some(&1) && env.contains_key(in_name) {\n"
                "                        let mut x = env.remove(in_name).unwrap();\n"
                "                        usage_count.remove(in_name);\n"
                "                        ops::softmax_inplace(&mut x, axis)?;\n",
             "                    let written_as_probs = self.fused_softmax.contains_key(in_name)\n"
             "                        && env.get(in_name).is_some_and(|x| softmax_axis_is_last(axis, x.shape().len()));\n"
             "                    if written_as_probs {\n"
             "                        // the head's MatMul wrote the probabilities\n"
             "                        usage_count.remove(in_name);\n"
             "                        env.remove(in_name).unwrap()\n"
             "                    } else if usage_count.get(in_name) == Some(&1) && env.contains_key(in_name) {\n"
             "                        let mut x = env.remove(in_name).unwrap();\n"
             "                        usage_count.remove(in_name);\n"
             "                        ops::softmax_inplace(&mut x, axis)?;\n")
    s = edit(s, "            env.insert(out_name.as_str(), out_tensor);\n",
             "            env.insert(out_name.as_str(), out_tensor);\n"
             "            if stop == Some(out_name.as_str()) {\n"
             "                let t = env.remove(out_name.as_str()).unwrap();\n"
             "                return Ok((t, profile_data));\n"
             "            }\n")
    s = edit(s, "/// Read the `group` attribute of `node` as a `usize`, rejecting zero and negatives.\n",
             "/// Whether a Softmax `axis` (negative counting from the end, as softmax_inplace takes it)\n"
             "/// is the last axis of a rank-`rank` tensor.\n"
             "fn softmax_axis_is_last(axis: isize, rank: usize) -> bool {\n"
             "    let r = rank as isize;\n"
             "    (if axis < 0 { axis + r } else { axis }) == r - 1\n"
             "}\n\n"
             "/// Read the `group` attribute of `node` as a `usize`, rejecting zero and negatives.\n")
    return s


def pipeline_rs(s):
    s = edit(s, "use crate::error::{OcrError, Result};\n",
             "use crate::error::{OcrError, Result};\nuse crate::ops::gpu_head::{GpuHead, RecHeadBackend};\n")
    s = edit(s, "    pub quantize_rec_head: bool,\n",
             "    pub quantize_rec_head: bool,\n"
             "    /// Where the recognition head (projection, softmax, CTC argmax) runs: the CPU\n"
             "    /// operators (default) or the HIP head on an MI355X.\n"
             "    pub rec_head_backend: RecHeadBackend,\n")
    s = edit(s, "            quantize_rec_head: false,\n",
             "            quantize_rec_head: false,\n            rec_head_backend: RecHeadBackend::Cpu,\n")
    s = edit(s, "        if config.quantize_rec_head {\n            rec_model.quantize_matmul_weights();\n        }\n",
             "        if config.quantize_rec_head {\n            rec_model.quantize_matmul_weights();\n        }\n"
             "        rec_model.attach_gpu_heads(config.rec_head_backend)?;\n")
    s = edit(s, "    pub fn enable_rec_quantization(&mut self) {\n        self.rec_model.quantize_matmul_weights();\n    }\n",
             "    pub fn enable_rec_quantization(&mut self) {\n        self.rec_model.quantize_matmul_weights();\n"
             "        // the HIP head follows the packed weight; on failure the CPU operators run it\n"
             "        if let Err(e) = self.rec_model.attach_gpu_heads(self.config.rec_head_backend) {\n"
             "            eprintln!(\"warning: HIP recognition head not rebuilt ({e}); the CPU head runs\");\n"
             "            let _ = self.rec_model.attach_gpu_heads(RecHeadBackend::Cpu);\n"
             "        }\n    }\n")
    s = edit(s, "        if boxes.len() == 1 {\n            return Ok(self\n",
             "        if let Some((head, head_input)) = self.rec_model.rec_head() {\n"
             "            return self.recognize_with_gpu_head(&rgb_img, boxes, use_cls, rec_input_name, head, head_input);\n"
             "        }\n\n"
             "        if boxes.len() == 1 {\n            return Ok(self\n")
    s = edit(s, "    /// Run full end-to-end OCR (detection + recognition)\n",
             "    /// recognize() with the HIP head: the rec graph runs up to the head's input for every\n"
             "    /// box (on the rec_pool, as before), the lines' [T_i, k] activations are packed back to\n"
             "    /// back, and one call (CtcDecoder::decode_page -> ppocr_rh_decode: projection, softmax\n"
             "    /// statistics, argmax and CTC collapse on the GPU) decodes the page.  Results match\n"
             "    /// recognize_single_box's: empty texts are dropped, boxes keep their order.\n"
             "    fn recognize_with_gpu_head(\n"
             "        &self,\n"
             "        rgb_img: &image::RgbImage,\n"
             "        boxes: &[TextBox],\n"
             "        use_cls: bool,\n"
             "        rec_input_name: &str,\n"
             "        head: &GpuHead,\n"
             "        head_input: &str,\n"
             "    ) -> Result<Vec<OcrResult>> {\n"
             "        use rayon::prelude::*;\n"
             "        let run = || -> Result<Vec<(Tensor, Option<u16>)>> {\n"
             "            boxes\n"
             "                .par_iter()\n"
             "                .map(|b| {\n"
             "                    let _guard = crate::tensor::ScopedDisableParallel::new();\n"
             "                    let mut patch = get_rotate_crop_image_rgb(rgb_img, &b.points);\n"
             "                    let angle = if use_cls { self.correct_orientation(&mut patch)? } else { None };\n"
             "                    let x = self.rec_preprocess.process(&patch)?;\n"
             "                    Ok((self.rec_model.forward_until(rec_input_name, x, head_input)?, angle))\n"
             "                })\n"
             "                .collect()\n"
             "        };\n"
             "        let lines = match self.rec_pool {\n"
             "            Some(ref pool) => pool.install(run)?,\n"
             "            None => run()?,\n"
             "        };\n"
             "        let k = head.k();\n"
             "        let mut line_off = vec![0i64];\n"
             "        let mut rows = Vec::new();\n"
             "        for (t, _) in &lines {\n"
             "            if t.shape().last() != Some(&k) {\n"
             "                return Err(OcrError::OperatorError {\n"
             "                    op: \"RecHeadHip\".into(),\n"
             "                    msg: format!(\"head input {:?}, expected [.., {}]\", t.shape(), k),\n"
             "                });\n"
             "            }\n"
             "            if t.is_contiguous() {\n"
             "                rows.extend_from_slice(t.as_slice());\n"
             "            } else {\n"
             "                rows.extend_from_slice(t.to_contiguous().as_slice());\n"
             "            }\n"
             "            line_off.push(line_off[line_off.len() - 1] + (t.numel() / k) as i64);\n"
             "        }\n"
             "        let page = Tensor::from_vec(&[rows.len() / k, k], rows)?;\n"
             "        let texts = self.ctc_decoder.decode_page(head, &page, &line_off)?;\n"
             "        Ok(boxes\n"
             "            .iter()\n"
             "            .zip(lines)\n"
             "            .zip(texts)\n"
             "            .filter(|(_, (text, _))| !text.is_empty())\n"
             "            .map(|((b, (_, angle)), (text, score))| OcrResult { points: b.points, text, score, angle })\n"
             "            .collect())\n"
             "    }\n\n"
             "    /// Run full end-to-end OCR (detection + recognition)\n")
    return s


def main(ref):
    out = os.path.join(HERE, "patches")
    os.makedirs(out, exist_ok=True)
    for rel, fn, name in (("src/engine/model.rs", model_rs, "engine_model.patch"),
                          ("src/pipeline.rs", pipeline_rs, "pipeline.patch")):
        orig = open(os.path.join(ref, rel)).read()
        with tempfile.TemporaryDirectory() as tmp:
            a = os.path.join(tmp, "a", rel)
            b = os.path.join(tmp, "b", rel)
            os.makedirs(os.path.dirname(a))
            os.makedirs(os.path.dirname(b))
            open(a, "w").write(orig)
            open(b, "w").write(fn(orig))
            d = subprocess.run(["diff", "-u", "a/" + rel, "b/" + rel], cwd=tmp, capture_output=True, text=True)
            assert d.returncode == 1, d.stderr
            text = "".join(l for l in d.stdout.splitlines(True))
            text = "\n".join(("--- a/" + rel if l.startswith("--- ") else "+++ b/" + rel if l.startswith("+++ ") else l)
                             for l in text.split("\n"))
            open(os.path.join(out, name), "w").write(text)
            print(name, text.count("\n@@"), "hunks")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
