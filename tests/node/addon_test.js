'use strict'
/*
 * The N-API addon and HipGpu, run by Node (CommonJS, Node 12). Usage:
 *   node addon_test.js cpu <gguf path> <onnx path>   (no GPU: sizes, errors, readers)
 *   node addon_test.js gpu <folder>                   (textures, reads, fences, a Q4_0 GEMV,
 *                                                      operands refused by size)
 * Assertions fail the process; a JSON summary of what was read goes to
 * stdout for the Python side to compare with its own readers.
 */
const assert = require('assert')
const fs = require('fs')
const path = require('path')

const hip = require(path.join(__dirname, '..', '..', 'webgllm_amd', 'node', 'index.js'))

function throwsGpu (fn, code, text) {
  let err = null
  try { fn() } catch (e) { err = e }
  assert.ok(err, 'expected a GpuError')
  // HipGpu's calls throw its GpuError class; the raw addon's errors carry the name
  assert.ok(err instanceof hip.GpuError || err.name === 'GpuError', `expected a GpuError, got ${err}`)
  assert.strictEqual(err.code, code)
  if (text) assert.ok(err.message.includes(text), err.message)
  return err
}

function cpu (ggufPath, onnxPath) {
  assert.ok(hip.version().includes('gfx950'))
  const C = hip.constants
  // src/weights.ts:153-178: 2048 x 2048 Q4_0 is 524,288 words and 131,072 halves
  assert.deepStrictEqual(hip.quantSizes(2048, 2048), { quants: 2048 * 2048 / 2, scales: 131072 * 2, zeros: 0 })
  assert.strictEqual(hip.quantSizes(4096, 4096, C.LAYOUT_ROWGROUP, C.ZERO_U8).zeros, 4096 * 128)
  assert.strictEqual(hip.quantSizes(4096, 4096, C.LAYOUT_Q4K, 0).quants, 4096 * 16 * 144)
  throwsGpu(() => hip.quantSizes(6, 32), 'WG_ERR_INVALID', 'multiple of 4')
  throwsGpu(() => hip.quantSizes(4, 32, C.LAYOUT_Q4K, 0), 'WG_ERR_INVALID', 'multiple of 256')
  throwsGpu(() => hip.quantSizes(4, 32, 9, 0), 'WG_ERR_UNSUPPORTED', 'unknown layout')
  assert.throws(() => hip.quantSizes('a', 32), TypeError)
  assert.throws(() => hip.addon.bufZero({}, {}), TypeError)
  const e = throwsGpu(() => hip.ggufHeader('/nonexistent/x.gguf'), 'WG_ERR_INVALID')
  assert.strictEqual(e.status, -1)
  throwsGpu(() => hip.onnxGraph('/nonexistent/x.onnx'), 'WG_ERR_INVALID')
  const g = hip.ggufHeader(ggufPath)
  const o = hip.onnxGraph(onnxPath)
  return {
    gguf: {
      version: g.version,
      dataOffset: g.dataOffset,
      tensors: g.tensors.map((t) => [t.name, t.dims, t.type, t.offset, t.bytes]),
      meta: g.meta
    },
    onnx: {
      name: o.name,
      nodes: o.nodes.map((n) => [n.name, n.opType, n.domain, n.inputs, n.outputs, Object.keys(n.attributes).sort()]),
      initializers: o.initializers.map((t) => [t.name, t.dims, t.dataType, t.location || null, t.offset === undefined ? null : t.offset, t.length === undefined ? null : t.length])
    }
  }
}

async function gpu (dir) {
  const GL = hip.GL
  const gpu = new hip.HipGpu(0)
  assert.ok(gpu.limits.computeUnits >= 1)
  const base = gpu.bytes
  // an RGBA32F texture, written whole, then a rectangle of it
  const W = 64
  const H = 16
  const px = new Float32Array(W * H * 4).map((_, i) => i * 0.5)
  const t = gpu.texture(GL.RGBA32F, W, H, { format: 0, type: 0, pixels: px })
  assert.strictEqual(gpu.bytes, base + W * H * 16)
  assert.deepStrictEqual(Array.from(gpu.readNow(t)), Array.from(px))
  const patch = new Float32Array(3 * 2 * 4).fill(-1)
  gpu.write(t, { x: 5, y: 7, width: 3, height: 2 }, { format: 0, type: 0, pixels: patch })
  const want = Float32Array.from(px)
  for (let r = 0; r < 2; r++) for (let c = 0; c < 3; c++) for (let k = 0; k < 4; k++) want[((7 + r) * W + 5 + c) * 4 + k] = -1
  // a pending read awaited across event-loop turns
  const full = await gpu.readStart(t)()
  assert.deepStrictEqual(Array.from(full), Array.from(want))
  const rect = await gpu.read(t, { x: 4, y: 6, width: 5, height: 4 })
  for (let r = 0; r < 4; r++) for (let c = 0; c < 5; c++) for (let k = 0; k < 4; k++) {
    assert.strictEqual(rect[(r * 5 + c) * 4 + k], want[((6 + r) * W + 4 + c) * 4 + k])
  }
  // a cancelled read can't be awaited; later reads still work
  const p = gpu.readStart(t)
  p.cancel()
  await assert.rejects(p(), /cancelled/)
  gpu.zero(t)
  assert.ok(gpu.readNow(t).every((v) => v === 0))
  gpu.delete(t)
  assert.strictEqual(gpu.bytes, base)
  throwsGpu(() => hip.addon.bufZero(gpu.ctx, t.tex), 'WG_ERR_DISPOSED')

  // a Q4_0 matrix from its GGUF blocks, repacked on the GPU, and a GEMV
  const meta = JSON.parse(fs.readFileSync(path.join(dir, 'gemv.json')))
  const { N, K, M } = meta
  const src = fs.readFileSync(path.join(dir, 'q4_0.bin'))
  const x16 = fs.readFileSync(path.join(dir, 'x16.bin'))
  const sizes = hip.quantSizes(N, K)
  const tsrc = gpu.texture(GL.R8UI, src.length, 1, { format: 0, type: 0, pixels: src })
  const w = {
    N, K, layout: hip.constants.LAYOUT_ROWGROUP, zero: hip.constants.ZERO_8,
    quants: gpu.texture(GL.RGBA32UI, sizes.quants / 16, 1),
    scales: gpu.texture(GL.R8UI, sizes.scales, 1)
  }
  gpu.ops.repack('q4_0', w, 0, N, tsrc)
  const tx = gpu.texture(GL.R8UI, x16.length, 1, { format: 0, type: 0, pixels: x16 })
  const ty = gpu.texture(GL.R32F, N, M)
  gpu.ops.gemv(w, tx, M, ty)
  const y = await gpu.read(ty)
  fs.writeFileSync(path.join(dir, 'y.bin'), Buffer.from(y.buffer))
  const ids = gpu.texture(GL.R32UI, M, 1)
  const scratch = gpu.texture(GL.R8UI, gpu.ops.argmaxScratchBytes(M, N), 1)
  gpu.ops.argmax(ty, M, N, ids, scratch)
  const picks = Array.from(new Int32Array(gpu.readNow(ids).buffer))
  const dq = gpu.texture(GL.R32F, K, 4)
  gpu.ops.dequant(w, 8, 4, dq)
  fs.writeFileSync(path.join(dir, 'dequant.bin'), Buffer.from(gpu.readNow(dq).buffer))
  // a Q4_K-records matrix: repacked from Q4_K blocks, its prompt halves kept
  const src4 = fs.readFileSync(path.join(dir, 'q4_k.bin'))
  const N4 = 64
  const s4 = hip.quantSizes(N4, K, hip.constants.LAYOUT_ROWGROUP, hip.constants.ZERO_Q4K)
  assert.strictEqual(s4.zeros, 0)
  assert.strictEqual(s4.quants + s4.scales, N4 * K / 256 * 144)
  const t4 = gpu.texture(GL.R8UI, src4.length, 1, { format: 0, type: 0, pixels: src4 })
  const w4 = {
    N: N4, K, layout: hip.constants.LAYOUT_ROWGROUP, zero: hip.constants.ZERO_Q4K,
    quants: gpu.texture(GL.RGBA32UI, s4.quants / 16, 1),
    scales: gpu.texture(GL.R8UI, s4.scales, 1)
  }
  gpu.ops.repack('q4_k', w4, 0, N4, t4)
  const halves = gpu.texture(GL.R8UI, N4 * K / 32 * 4, 1)
  gpu.ops.q4kRecordHalves(w4, halves, gpu.view(halves, N4 * K / 32 * 2))
  fs.writeFileSync(path.join(dir, 'q4k_halves.bin'), Buffer.from(gpu.readNow(halves).buffer))
  const dq4 = gpu.texture(GL.R32F, K, 4)
  gpu.ops.dequant(w4, 4, 4, dq4)
  fs.writeFileSync(path.join(dir, 'q4k_dequant.bin'), Buffer.from(gpu.readNow(dq4).buffer))
  throwsGpu(() => gpu.ops.q4kRecordHalves(w4, gpu.texture(GL.R8UI, 16, 1), halves), 'WG_ERR_INVALID', 'scales')
  throwsGpu(() => gpu.ops.q4kRecordHalves(w, halves, halves), 'WG_ERR_INVALID')
  // bad shapes are refused before any launch
  throwsGpu(() => gpu.ops.gemv(Object.assign({}, w, { K: K + 1 }), tx, M, ty), 'WG_ERR_INVALID')
  // operands smaller than their shapes imply are refused before any launch
  // (the device would otherwise read or write past them)
  const small = gpu.texture(GL.R32F, 4, 1)
  throwsGpu(() => gpu.ops.gemv(w, tx, M, small), 'WG_ERR_INVALID', 'y: ')
  throwsGpu(() => gpu.ops.gemv(w, small, M, ty), 'WG_ERR_INVALID', 'x: ')
  throwsGpu(() => gpu.ops.gemv(w, tx, M, ty, { mode: hip.constants.EPI_STORE, residual: small, ldResidual: N }), 'WG_ERR_INVALID', 'residual')
  throwsGpu(() => gpu.ops.gemv(Object.assign({}, w, { quants: small }), tx, M, ty), 'WG_ERR_INVALID', 'quants')
  throwsGpu(() => gpu.ops.gemv(w, gpu.view(tx, x16.length - 16), M, ty), 'WG_ERR_INVALID', 'offset')
  throwsGpu(() => gpu.ops.repack('q4_0', w, 0, N, small), 'WG_ERR_INVALID', 'src')
  throwsGpu(() => gpu.ops.repack('q4_0', w, 0, 4, tsrc, Int32Array.from([0, 1, 2, N])), 'WG_ERR_INVALID', 'srcRows[3]')
  throwsGpu(() => gpu.ops.argmax(ty, M, N, ids, small), 'WG_ERR_INVALID', 'scratch')
  throwsGpu(() => gpu.ops.dequant(w, 0, 4, small), 'WG_ERR_INVALID', 'out')
  const shape = { heads: 4, kvHeads: 2, headDim: 64 }
  throwsGpu(() => gpu.ops.attnDecode(small, 1, shape, small, small, small, 16, small, small), 'WG_ERR_INVALID')
  throwsGpu(() => gpu.ops.shortConv(small, 1, 64, 3, small, small, small, null, small), 'WG_ERR_INVALID', 'bcx')
  // a read's bytes are the fence's own: another count is refused before the copy
  const rf = hip.addon.readStart(gpu.ctx, ty.tex, 0, 64)
  throwsGpu(() => hip.addon.readFinish(rf, 4096), 'WG_ERR_INVALID', 'holds 64 bytes')
  assert.strictEqual(hip.addon.readFinish(rf).byteLength, 64)
  // plain fences (PacedGpu.fence / fenceReady / wait / deleteFence)
  const f1 = gpu.fence()
  await gpu.wait(f1)
  const f2 = gpu.fence()
  gpu.deleteFence(f2)
  throwsGpu(() => hip.addon.fenceReady(f2), 'WG_ERR_DISPOSED')
  assert.strictEqual(gpu.readBack(), true)
  // the device still works after the refusals: the same GEMV again
  gpu.ops.gemv(w, tx, M, ty)
  const y2 = await gpu.read(ty)
  assert.deepStrictEqual(Array.from(y2), Array.from(y))
  assert.ok(gpu.limits.maxTextureSize >= 1 << 20 && gpu.limits.maxTextureUnits >= 16)
  const staging = hip.addon.staging(gpu.ctx)
  gpu.dispose()
  assert.strictEqual(hip.addon.bytesLive(gpu.ctx), 0)
  throwsGpu(() => hip.addon.finish(gpu.ctx), 'WG_ERR_DISPOSED')
  return { picks, staging }
}

async function main () {
  const mode = process.argv[2]
  const out = mode === 'cpu' ? cpu(process.argv[3], process.argv[4]) : await gpu(process.argv[3])
  process.stdout.write(JSON.stringify(out) + '\n')
}

main().catch((e) => {
  console.error(e && e.stack ? e.stack : e)
  process.exit(1)
})
