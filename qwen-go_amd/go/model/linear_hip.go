//go:build qmoe

// linear_hip.go -- the dense projections on the device (qmoe_linear_*,
// include/qmoe.h): linear.matvec / mat2D / proj (model/model.go:131-205) and
// quantLinear.forward (model/moe.go:159-162) with outputs bit-identical to the
// reference's sequential f32 sums, and greedy decode's argmax
// (model/model.go:652-660) over the LM head's logits (model.go:519-525).
package model

/*
#include "qmoe.h"
*/
import "C"

import (
	"fmt"
	"unsafe"
)

// linearDev is the device copy of one projection.
type linearDev struct {
	h       *C.qmoe_linear
	out, in int
}

func linearErr(h *C.qmoe_linear, st C.qmoe_status, what string) error {
	return fmt.Errorf("qmoe linear %s: %s: %s", what, C.GoString(C.qmoe_status_string(st)),
		C.GoString(C.qmoe_linear_last_error(h)))
}

// newLinearDev uploads l (or its quantLinear q) to device `device`.
func newLinearDev(l *linear, q *quantLinear, out, in, device int) (*linearDev, error) {
	w, s, f, err := projWeights(l, q)
	if err != nil {
		return nil, err
	}
	var h *C.qmoe_linear
	if st := C.qmoe_linear_create(C.int32_t(out), C.int32_t(in), f, C.int32_t(device), &h); st != C.QMOE_OK {
		return nil, linearErr(nil, st, "create")
	}
	if st := C.qmoe_linear_set(h, w, s); st != C.QMOE_OK {
		e := linearErr(h, st, "upload")
		C.qmoe_linear_destroy(h)
		return nil, e
	}
	return &linearDev{h: h, out: out, in: in}, nil
}

// matvec is linear.matvec on the device: y = x @ W^T for T rows of x.
func (d *linearDev) matvec(x []float32, T int) []float32 {
	if len(x) != T*d.in {
		panic(fmt.Sprintf("qmoe linear: %d values for %d rows of %d", len(x), T, d.in))
	}
	y := make([]float32, T*d.out)
	st := C.qmoe_linear_forward(d.h, (*C.float)(unsafe.Pointer(&x[0])), C.int32_t(T), (*C.float)(unsafe.Pointer(&y[0])))
	if st != C.QMOE_OK {
		panic(linearErr(d.h, st, "forward"))
	}
	return y
}

// greedy returns argmax(x @ W^T) for one token without copying the logits
// back: the LM head of greedy decode.
func (d *linearDev) greedy(x []float32) int {
	if len(x) != d.in {
		panic(fmt.Sprintf("qmoe linear: %d values, want %d", len(x), d.in))
	}
	var tok C.int32_t
	st := C.qmoe_linear_greedy(d.h, (*C.float)(unsafe.Pointer(&x[0])), 1, &tok, nil)
	if st != C.QMOE_OK {
		panic(linearErr(d.h, st, "greedy"))
	}
	return int(tok)
}

func (d *linearDev) close() {
	if d != nil && d.h != nil {
		C.qmoe_linear_destroy(d.h)
		d.h = nil
	}
}
