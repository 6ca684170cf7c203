//go:build qmoe

// moe_hip.go -- the cgo seam between qwen-go's moeMLP and libqmoe.so (the
// MI355X MoE block, include/qmoe.h).  Copy this file and moe_hip_stub.go into
// qwen-go's model/ directory and build with `-tags qmoe`, with
//   CGO_CFLAGS="-I<this repo>/include"
//   CGO_LDFLAGS="-L<this repo>/qwen-go_amd -lqmoe -Wl,-rpath,<this repo>/qwen-go_amd"
// The three small edits to existing files (a field in moeMLP, the first lines
// of moeMLP.forward, the batched branch of decodeLayers and the upload after
// loading) are listed in INTEGRATION.md.
package model

/*
#cgo LDFLAGS: -lqmoe
#include <stdlib.h>
#include "qmoe.h"
*/
import "C"

import (
	"encoding/json"
	"fmt"
	"os"
	"path/filepath"
	"strings"
	"unsafe"

	"tinyqwengo/safetensors"
)

// qmoeDev is the device copy of one moeMLP (a qmoe_layer handle).
type qmoeDev struct {
	h    *C.qmoe_layer
	norm bool // post-attention norm uploaded (forwardResidualT)
}

// qmoeErr formats a failed call.  The handle's message is copied into a Go
// string here, so call it before qmoe_destroy.
func qmoeErr(h *C.qmoe_layer, st C.qmoe_status, what string) error {
	return fmt.Errorf("qmoe %s: %s: %s", what, C.GoString(C.qmoe_status_string(st)),
		C.GoString(C.qmoe_last_error(h)))
}

// projWeights returns the host storage of one projection as the loader filled
// it -- a quantLinear from installQuant (model/load.go:646-664; its scales are
// []float32, as qwen-quant writes them), raw bf16 bytes from setLinear in raw
// mode, or f32 weights -- and the qmoe format that describes it.  It never
// indexes an empty slice.
func projWeights(l *linear, q *quantLinear) (w, s unsafe.Pointer, f C.int32_t, err error) {
	switch {
	case q != nil:
		if len(q.qweight) == 0 || len(q.scale) == 0 {
			return nil, nil, 0, fmt.Errorf("quantised projection without codes or scales")
		}
		switch q.bits {
		case 8:
			f = C.QMOE_INT8G32_F32S
		case 4:
			f = C.QMOE_INT4G32_F32S
		default:
			return nil, nil, 0, fmt.Errorf("quantised projection with %d bits", q.bits)
		}
		return unsafe.Pointer(&q.qweight[0]), unsafe.Pointer(&q.scale[0]), f, nil
	case len(l.raw) > 0:
		return unsafe.Pointer(&l.raw[0]), nil, C.QMOE_BF16, nil
	case len(l.w) > 0:
		return unsafe.Pointer(&l.w[0]), nil, C.QMOE_F32, nil
	}
	return nil, nil, 0, fmt.Errorf("projection has no weights")
}

// uploadQmoe copies m's weights to device `device` once, after loadMLP and
// installQuant have filled m.  selectScope 0 keeps the reference's selection
// (model/moe.go:45-53); nExperts gives true top-k.
func (m *moeMLP) uploadQmoe(device int, selectScope int) (err error) {
	rw, rs, rfmt, err := projWeights(&m.gate, m.routerQuant)
	if err != nil {
		return fmt.Errorf("qmoe router: %w", err)
	}
	desc := C.qmoe_desc{
		hidden: C.int32_t(m.nEmbed), n_experts: C.int32_t(m.nExperts), top_k: C.int32_t(m.topK),
		moe_inter: C.int32_t(m.nMoeMlp), select_scope: C.int32_t(selectScope), device: C.int32_t(device),
		router_fmt: rfmt, expert_fmt: C.QMOE_BF16, shared_fmt: C.QMOE_BF16,
	}
	var gu, dn, gus, dns unsafe.Pointer
	switch {
	case m.packed != nil:
		p := m.packed
		if len(p.gateUp) == 0 || len(p.gateUpScale) == 0 || len(p.down) == 0 || len(p.downScale) == 0 {
			return fmt.Errorf("qmoe: packed experts without codes or scales")
		}
		gu, gus = unsafe.Pointer(&p.gateUp[0]), unsafe.Pointer(&p.gateUpScale[0])
		dn, dns = unsafe.Pointer(&p.down[0]), unsafe.Pointer(&p.downScale[0])
		desc.expert_fmt = C.QMOE_INT8G32
		if p.bits == 4 {
			desc.expert_fmt = C.QMOE_INT4G32
		}
	case len(m.gateUpRaw) > 0 && len(m.downRaw) > 0:
		gu, dn = unsafe.Pointer(&m.gateUpRaw[0]), unsafe.Pointer(&m.downRaw[0])
	case len(m.gateUpW) > 0 && len(m.downW) > 0:
		gu, dn = unsafe.Pointer(&m.gateUpW[0]), unsafe.Pointer(&m.downW[0])
		desc.expert_fmt = C.QMOE_F32
	default:
		return fmt.Errorf("qmoe: experts not loaded")
	}
	type projection struct{ w, s unsafe.Pointer }
	var sh [3]projection
	if m.shared != nil {
		desc.shared_inter = C.int32_t(m.shared.nMlp)
		var f [3]C.int32_t
		for i, p := range []struct {
			l *linear
			q *quantLinear
		}{{&m.shared.gate, m.shared.gateQuant}, {&m.shared.up, m.shared.upQuant}, {&m.shared.down, m.shared.downQuant}} {
			if sh[i].w, sh[i].s, f[i], err = projWeights(p.l, p.q); err != nil {
				return fmt.Errorf("qmoe shared expert: %w", err)
			}
		}
		if f[0] != f[1] || f[0] != f[2] {
			return fmt.Errorf("qmoe: shared expert projections in different formats")
		}
		desc.shared_fmt = f[0]
		if len(m.sharedGate) != m.nEmbed {
			return fmt.Errorf("qmoe: shared expert gate has %d values, want %d", len(m.sharedGate), m.nEmbed)
		}
	}
	var h *C.qmoe_layer
	if st := C.qmoe_create(&desc, &h); st != C.QMOE_OK {
		return qmoeErr(nil, st, "create")
	}
	fail := func(st C.qmoe_status, what string) error {
		e := qmoeErr(h, st, what) // read the message before the handle goes
		C.qmoe_destroy(h)
		return e
	}
	if st := C.qmoe_set_router(h, rw, rs); st != C.QMOE_OK {
		return fail(st, "router")
	}
	if st := C.qmoe_set_experts(h, gu, gus, dn, dns); st != C.QMOE_OK {
		return fail(st, "experts")
	}
	if m.shared != nil {
		st := C.qmoe_set_shared(h, sh[0].w, sh[0].s, sh[1].w, sh[1].s, sh[2].w, sh[2].s,
			(*C.float)(unsafe.Pointer(&m.sharedGate[0])))
		if st != C.QMOE_OK {
			return fail(st, "shared")
		}
	}
	m.dev = &qmoeDev{h: h}
	return nil
}

// forwardQmoe is the body of moeMLP.forward when m.dev is set: one token.
func (m *moeMLP) forwardQmoe(x []float32) []float32 {
	return m.forwardT(x, 1)
}

// forwardT runs T tokens (x is (T, nEmbed), row-major) in one call: the
// batched seam that decodeLayers uses through batchMixer.  Each row of the
// result is moeMLP.forward of that row of x.
func (m *moeMLP) forwardT(x []float32, T int) []float32 {
	if m.dev == nil {
		out := make([]float32, 0, T*m.nEmbed)
		for t := 0; t < T; t++ {
			out = append(out, m.forward(x[t*m.nEmbed:(t+1)*m.nEmbed])...)
		}
		return out
	}
	if len(x) != T*m.nEmbed {
		panic(fmt.Sprintf("qmoe forward: %d values for %d tokens of %d", len(x), T, m.nEmbed))
	}
	out := make([]float32, T*m.nEmbed)
	st := C.qmoe_forward(m.dev.h, (*C.float)(unsafe.Pointer(&x[0])), C.int32_t(T),
		(*C.float)(unsafe.Pointer(&out[0])), nil, nil)
	if st != C.QMOE_OK {
		panic(qmoeErr(m.dev.h, st, "forward"))
	}
	return out
}

// setPostNormQmoe uploads the block's post-attention GemmaRMSNorm weight and
// eps (block.postAttentionLayernorm, float32(cfg.RmsNormEps)) for
// forwardResidualT.
func (m *moeMLP) setPostNormQmoe(w []float32, eps float32) error {
	if m.dev == nil {
		return fmt.Errorf("qmoe: no device copy")
	}
	if len(w) != m.nEmbed {
		return fmt.Errorf("qmoe: post-attention norm has %d values, want %d", len(w), m.nEmbed)
	}
	if st := C.qmoe_set_post_norm(m.dev.h, (*C.float)(unsafe.Pointer(&w[0])), C.float(eps)); st != C.QMOE_OK {
		return qmoeErr(m.dev.h, st, "post-attention norm")
	}
	m.dev.norm = true
	return nil
}

// forwardResidualT is decodeLayers' whole MLP step for T tokens, in place on
// the residual stream x (T, nEmbed): x[t] += forward(gemmaRMSNorm(x[t]))
// (model/model.go:506-517), with the norm and the residual add on the device.
func (m *moeMLP) forwardResidualT(x []float32, T int) {
	if len(x) != T*m.nEmbed {
		panic(fmt.Sprintf("qmoe residual forward: %d values for %d tokens of %d", len(x), T, m.nEmbed))
	}
	st := C.qmoe_forward_residual(m.dev.h, (*C.float)(unsafe.Pointer(&x[0])), C.int32_t(T), nil, nil)
	if st != C.QMOE_OK {
		panic(qmoeErr(m.dev.h, st, "residual forward"))
	}
}

// packedExperts are the stacked routed experts as stored by experts_file.py:
// <base>.qweight I8 (E, rows, K) int8 codes or (E, rows, K/2) int4 pairs, and
// <base>.scale F16 (E, rows, K/32).  The slices alias the shard's mmap.
type packedExperts struct {
	bits                int
	gateUp, gateUpScale []byte
	down, downScale     []byte
}

// packedManifest is quant.json with the keys experts_file.py adds; the
// reference's quantManifest ignores them.
type packedManifest struct {
	Bits             int      `json:"bits"`
	Experts          []string `json:"experts"`
	ExpertScaleDtype string   `json:"expert_scale_dtype"`
}

// loadPackedExperts attaches the packed experts of a quantised directory to
// the model's moeMLP blocks.  Call it after FromPretrained (whose shard mmaps
// in m.closers stay open) and before uploadQmoe; a directory without
// "experts" in quant.json is left alone.
func (m *model) loadPackedExperts(dir string) error {
	raw, err := os.ReadFile(filepath.Join(dir, "quant.json"))
	if err != nil {
		return nil // not a quantised directory
	}
	var man packedManifest
	if err := json.Unmarshal(raw, &man); err != nil {
		return err
	}
	if len(man.Experts) == 0 {
		return nil
	}
	if man.Bits != 8 && man.Bits != 4 {
		return fmt.Errorf("packed experts with %d bits", man.Bits)
	}
	if man.ExpertScaleDtype != "" && man.ExpertScaleDtype != "F16" {
		return fmt.Errorf("packed expert scales %q (only F16 is defined)", man.ExpertScaleDtype)
	}
	shards, _ := filepath.Glob(filepath.Join(dir, "*.safetensors"))
	for _, shard := range shards {
		f, closer, err := openShard(shard)
		if err != nil {
			return err
		}
		m.closers = append(m.closers, closer)
		for _, key := range f.Keys() {
			if !strings.HasSuffix(key, ".qweight") || !strings.Contains(key, ".mlp.experts.") {
				continue
			}
			base := strings.TrimSuffix(key, ".qweight")
			qw, qshape, qdt, err := f.Raw(key)
			if err != nil {
				return err
			}
			sc, sshape, sdt, err := f.Raw(base + ".scale")
			if err != nil {
				return err
			}
			if qdt != safetensors.I8 || sdt != safetensors.F16 || len(qshape) != 3 || len(sshape) != 3 {
				return fmt.Errorf("%s: packed experts must be I8 (E, rows, K) + F16 scales", base)
			}
			flat := renameKey(base)
			layer, which, err := packedTarget(flat)
			if err != nil {
				return err
			}
			if layer < 0 || layer >= len(m.layers) {
				return fmt.Errorf("%s: layer %d out of range", base, layer)
			}
			moe, ok := m.layers[layer].mlp.(*moeMLP)
			if !ok {
				return fmt.Errorf("%s: layer %d has no MoE block", base, layer)
			}
			if moe.packed == nil {
				moe.packed = &packedExperts{bits: man.Bits}
			}
			k := qshape[2]
			if man.Bits == 4 {
				k *= 2
			}
			if sshape[0] != qshape[0] || sshape[1] != qshape[1] || sshape[2]*32 != k {
				return fmt.Errorf("%s: scale shape %v does not match codes %v", base, sshape, qshape)
			}
			if which == "gate_up_proj" {
				moe.packed.gateUp, moe.packed.gateUpScale = qw, sc
			} else {
				moe.packed.down, moe.packed.downScale = qw, sc
			}
		}
	}
	return nil
}

// packedTarget splits "layers.N.mlp.experts.<which>" into N and which.
func packedTarget(flat string) (int, string, error) {
	var layer int
	var which string
	rest := strings.TrimPrefix(flat, "layers.")
	dot := strings.Index(rest, ".")
	if dot <= 0 || !strings.HasPrefix(flat, "layers.") {
		return 0, "", fmt.Errorf("unsupported packed target %q", flat)
	}
	for _, c := range rest[:dot] {
		if c < '0' || c > '9' {
			return 0, "", fmt.Errorf("bad layer index in %q", flat)
		}
		layer = layer*10 + int(c-'0')
	}
	which = strings.TrimPrefix(rest[dot:], ".mlp.experts.")
	if which != "gate_up_proj" && which != "down_proj" {
		return 0, "", fmt.Errorf("unsupported packed target %q", flat)
	}
	return layer, which, nil
}

// closeQmoe releases the device copy.
func (m *moeMLP) closeQmoe() {
	if m.dev != nil {
		C.qmoe_destroy(m.dev.h)
		m.dev = nil
	}
}
