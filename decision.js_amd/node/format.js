"use strict";
/* Model files on the Node host: manifest.json + weights.bin in the decision.js format (export_common.py:17-61;
 * manifest {format: "d1.js/1", config, tensors{dtype, shape, offset, bytes, scales, scales_bytes}, bytes}),
 * read the way loadWeights does (gpu.ts:57-88): the manifest, then each tensor's byte ranges through a
 * `fetch` that honours `Range: bytes=a-b`, six tensors in flight, a length check per read, and a refusal
 * when a tensor is larger than the device.
 *
 * Node 12 has no fetch: fileFetch(base) is the file-backed one a host passes as opts.fetch (any fetch with
 * Range support works, e.g. over HTTP). */
const fs = require("fs");
const path = require("path");
const { Context } = require("./dj");

const FORMAT = "d1.js/1";

/** A fetch over local files: `url` is a path; a Range header reads just those bytes. */
function fileFetch() {
  return async (url, init) => {
    const range = init && init.headers && (init.headers.Range || init.headers.range);
    const fd = fs.openSync(url, "r");
    try {
      let buf;
      if (range) {
        const m = /^bytes=(\d+)-(\d+)$/.exec(range);
        if (!m) throw new Error(`decision.js: unsupported Range header ${range}`);
        const a = Number(m[1]), b = Number(m[2]);
        buf = Buffer.alloc(b - a + 1);
        let got = 0;
        while (got < buf.length) {
          const n = fs.readSync(fd, buf, got, buf.length - got, a + got);
          if (n === 0) break;
          got += n;
        }
        buf = buf.subarray(0, got);
      } else {
        buf = fs.readFileSync(url);
      }
      return {
        ok: true,
        arrayBuffer: async () => buf.buffer.slice(buf.byteOffset, buf.byteOffset + buf.length),
        json: async () => JSON.parse(buf.toString("utf8")),
      };
    } finally {
      fs.closeSync(fd);
    }
  };
}

/** The manifest and every tensor of `base` on the device: {ctx, m, w}. Quantized tensors become Weight
 * (layout(name, info) picks the device layout), f16/f32 ones DevBuf (with the host copy as .host).
 * opts: fetch, device (a Context), onProgress(loaded, total). */
async function loadWeights(base, opts, layout) {
  opts = opts || {};
  const get = opts.fetch || fileFetch();
  const sep = base.endsWith("/") ? "" : "/";
  const m = await (await get(`${base}${sep}manifest.json`)).json();
  if (m.format !== FORMAT) throw new Error(`decision.js: ${base}${sep}manifest.json is not a ${FORMAT} manifest`);
  const ctx = opts.device || new Context(0);
  const names = Object.keys(m.tensors);
  const limit = ctx.info().memory;
  const largest = Math.max(...names.map((n) => m.tensors[n].bytes));
  if (largest > limit) throw new Error(`decision.js: this GPU holds ${(limit / 1e6).toFixed(0)} MB, this model needs a ${(largest / 1e6).toFixed(0)} MB tensor`);
  let loaded = 0;
  const range = async (offset, bytes) => {
    const res = await get(`${base}${sep}weights.bin`, { headers: { Range: `bytes=${offset}-${offset + bytes - 1}` } });
    const data = new Uint8Array(await res.arrayBuffer());
    if (data.byteLength !== bytes) throw new Error(`decision.js: range read returned ${data.byteLength} bytes, wanted ${bytes} (does the server support Range requests?)`);
    loaded += bytes;
    if (opts.onProgress) opts.onProgress(loaded, m.bytes);
    return data;
  };
  const w = {};
  for (let i = 0; i < names.length; i += 6) {
    await Promise.all(names.slice(i, i + 6).map(async (name) => {
      const t = m.tensors[name];
      if (t.dtype === "q4" || t.dtype === "q8") {
        const codes = await range(t.offset, t.bytes);
        const sraw = await range(t.scales, t.scales_bytes);
        const scales = new Uint16Array(sraw.buffer, sraw.byteOffset, sraw.byteLength / 2);
        const [N, K] = t.shape;
        w[name] = ctx.weightQ(codes, scales, N, K, t.dtype === "q8" ? 8 : 4, layout(name, t));
      } else {
        const raw = await range(t.offset, t.bytes);
        const host = t.dtype === "f16" ? new Uint16Array(raw.buffer, raw.byteOffset, raw.byteLength / 2)
          : new Float32Array(raw.buffer, raw.byteOffset, raw.byteLength / 4);
        const b = ctx.array(host);
        b.host = host;
        w[name] = b;
      }
    }));
  }
  // f32 tensors read on the host (the manifest's "host" list: EmbeddingGemma 2's decision head, eg2-engine.ts:46-50)
  const host = {};
  for (const [name, t] of Object.entries(m.host || {})) {
    const raw = await range(t.offset, t.bytes);
    host[name] = new Float32Array(raw.buffer, raw.byteOffset, raw.byteLength / 4);
  }
  return { ctx, m, w, host };
}

function loadManifestSync(base) {
  return JSON.parse(fs.readFileSync(path.join(base, "manifest.json"), "utf8"));
}

module.exports = { FORMAT, fileFetch, loadWeights, loadManifestSync };
